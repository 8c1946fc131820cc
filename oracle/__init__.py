"""CPU parity oracle for the fused quantized-MoE decode path.

TEST INFRASTRUCTURE ONLY.  Nothing in ``zmlx_amd`` imports this package; only
``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may use it, and only as the checker / the timed CPU baseline,
never as a code path of the product.

Contents
--------
``moe_oracle``  numpy restatement of MLX's *unpatched* MoE-block arithmetic
                (the parity target named by the reference's tests), with
                bf16 rounding emulated at every point MLX rounds.
``moe_ref.cpp`` the same restatement in C++ (OpenMP) for the CPU baseline
                timing and as a second, independently written implementation
                that the numpy one is cross-checked against.

Parity pins (what each function is checked against, all in ``tests/``):
closed forms (affine / mxfp4 dequant, exhaustive), the reference's known
answers (router tie-break and group selection, top-2 selection), brute force
on tiny inputs (top-k), and float64 recomputation for the GEMV stages.
"""
