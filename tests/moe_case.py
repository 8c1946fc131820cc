"""Seeded synthetic MoE weights/inputs shared by the tests (numpy side) and
helpers to move them onto the GPU as the library's layouts."""

from __future__ import annotations

from dataclasses import dataclass, field

import numpy as np

from oracle import moe_oracle as O


@dataclass
class Bank:
    """One stacked expert projection [E, N, K] in MLX layout."""

    w: np.ndarray          # uint32 [E, N, K/8]
    s: np.ndarray          # float32 (bf16 values) [E, N, K/gs]   or uint8 e8m0 [E, N, K/32]
    b: np.ndarray | None   # float32 (bf16 values) or None (mxfp4)
    mode: str = "affine"
    group_size: int = 64

    def deq(self, e: int) -> np.ndarray:
        return O.dequant(self.w[e], self.s[e], None if self.b is None else self.b[e],
                         group_size=self.group_size, mode=self.mode)

    def as_tuple(self):
        return (self.w, self.s, self.b)

    def torch(self, dev):
        import torch

        w = torch.from_numpy(np.ascontiguousarray(self.w)).to(dev)
        if self.mode == "affine":
            s = torch.from_numpy(np.ascontiguousarray(self.s)).to(torch.bfloat16).to(dev)
            b = torch.from_numpy(np.ascontiguousarray(self.b)).to(torch.bfloat16).to(dev)
        else:
            s = torch.from_numpy(np.ascontiguousarray(self.s)).to(dev)
            b = None
        return w, s, b


def seed_of(label: str) -> int:
    """Stable per-case seed (Python's str hash is randomised per process)."""
    import zlib

    return zlib.crc32(label.encode())


def make_bank(rng, E, N, K, *, mode="affine", group_size=64, std=0.02) -> Bank:
    w = (rng.standard_normal((E, N, K), dtype=np.float32) * std).astype(np.float32)
    w = O.bf16_round(w)
    if mode == "affine":
        q, s, b = O.quantize_affine(w, group_size=group_size, bits=4)
        return Bank(q, s, b, "affine", group_size)
    q, e = O.quantize_mxfp4(w)
    return Bank(q, e, None, "mxfp4", 32)


def bf16_randn(rng, shape, scale=1.0) -> np.ndarray:
    return O.bf16_round(rng.standard_normal(shape, dtype=np.float32) * np.float32(scale))


def to_bf16(a, dev):
    import torch

    return torch.from_numpy(np.ascontiguousarray(np.asarray(a, np.float32))).to(torch.bfloat16).to(dev)


def from_dev(t) -> np.ndarray:
    import torch

    if t.dtype == torch.bfloat16:
        return t.float().cpu().numpy()
    return t.cpu().numpy()


def qmm_exact(x, bank: Bank, lhs, rhs):
    """float64 exact value and abs-sum sum_i |w_i x_i| for every output of a
    gather_qmm (x [Bx, M, K]) -> two float64 arrays [P, M, N]."""
    vals, absd = [], []
    for li, ri in zip(np.asarray(lhs).reshape(-1), np.asarray(rhs).reshape(-1)):
        wd = bank.deq(int(ri)).astype(np.float64)
        xm = np.asarray(x[int(li)], np.float64)
        vals.append(xm @ wd.T)
        absd.append(np.abs(xm) @ np.abs(wd).T)
    return np.stack(vals), np.stack(absd)


def check_gemv_bound(got, exact, absdot, rel=2.0**-16):
    """Forward-error bound of a bf16-output GEMV: the result is the bf16
    rounding of a value within rel*sum|w x| of the exact dot product, so
    |got - exact| <= 0.5 ulp_bf16(got) + rel*sum|w x|; and >= 99% of outputs
    equal the correctly rounded exact value."""
    got = np.asarray(got, np.float64)
    # bf16 ulp of |got| = 2^(floor(log2|got|) - 7) = 2^(frexp exponent - 8)
    ulp = np.ldexp(1.0, np.frexp(np.maximum(np.abs(got), 2.0**-126))[1] - 8)
    err = np.abs(got - exact)
    bound = 0.5 * ulp + rel * absdot
    assert (err <= bound).all(), f"max err/bound {(err / bound).max():.3f}"
    exact_bf16 = O._f64_to_bf16(exact)
    frac = float((exact_bf16 == got.astype(np.float32)).mean())
    assert frac >= 0.99, f"correctly-rounded fraction {frac:.4f}"
