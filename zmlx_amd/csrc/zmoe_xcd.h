// XCD-partitioned single-launch kernel (decode1x.hip: one token with 8
// units): MI355X's XCD layout, the loads that read words other CUs of the
// same XCD stored, and the host-side check of how workgroups are dealt to
// the XCDs.
#pragma once

#include "zmoe_fused.h"

namespace zmoe {

constexpr int kNX = 8;                        // XCDs
constexpr int kXG = 256;                      // workgroups = CUs of MI355X
constexpr int kXWX = kXG / kNX * kFWaves;     // waves per XCD
constexpr int kXH = 2048;                     // hidden size

__host__ __device__ constexpr int cgcd(int a, int b) { return b == 0 ? a : cgcd(b, a % b); }

__device__ __forceinline__ int xcc_id() {
  // HW_REG_XCC_ID (hardware register 20), bits [3:0]
  return static_cast<int>(__builtin_amdgcn_s_getreg((3 << 11) | (0 << 6) | 20) & 0xF);
}

// Loads for words that other CUs of this XCD stored with ordinary stores
// (XCD-local exchange): the sc0 nt cache policy skips the CU's L1 and is
// served by the XCD's L2, where those stores land.  (Loads that do not skip
// L1 can keep returning a stale line; device-scope loads also see the words
// but take about twice as long under streaming load.)  The compiler's wait
// counts do not cover these loads, so each waits for its own results, and
// with them for every load the wave issued before.
template <int P>
__device__ __forceinline__ void xcd_load_row(const uint32_t* lg, int E, uint32_t (&wd)[P]) {
  const int lane = __lane_id();
  const uint32_t* a0 = lg + min(lane, E - 1);
  if constexpr (P == 1) {
    asm volatile("global_load_dword %0, %1, off sc0 nt\n\ts_waitcnt vmcnt(0)" : "=v"(wd[0]) : "v"(a0) : "memory");
  } else if constexpr (P == 2) {
    const uint32_t* a1 = lg + min(lane + 64, E - 1);
    asm volatile("global_load_dword %0, %2, off sc0 nt\n\tglobal_load_dword %1, %3, off sc0 nt\n\ts_waitcnt vmcnt(0)"
                 : "=&v"(wd[0]), "=&v"(wd[1])
                 : "v"(a0), "v"(a1)
                 : "memory");
  } else {
    static_assert(P == 4, "route slots");
    const uint32_t* a1 = lg + min(lane + 64, E - 1);
    const uint32_t* a2 = lg + min(lane + 128, E - 1);
    const uint32_t* a3 = lg + min(lane + 192, E - 1);
    asm volatile(
        "global_load_dword %0, %4, off sc0 nt\n\tglobal_load_dword %1, %5, off sc0 nt\n\t"
        "global_load_dword %2, %6, off sc0 nt\n\tglobal_load_dword %3, %7, off sc0 nt\n\ts_waitcnt vmcnt(0)"
        : "=&v"(wd[0]), "=&v"(wd[1]), "=&v"(wd[2]), "=&v"(wd[3])
        : "v"(a0), "v"(a1), "v"(a2), "v"(a3)
        : "memory");
  }
}
__device__ __forceinline__ void xcd_load_2x128(const uint32_t* ptr, uint4& a, uint4& b) {
  asm volatile("global_load_dwordx4 %0, %2, off sc0 nt\n\tglobal_load_dwordx4 %1, %2, off offset:16 sc0 nt\n\ts_waitcnt vmcnt(0)"
               : "=&v"(a), "=&v"(b)
               : "v"(ptr)
               : "memory");
}

// Spin limit of this kernel's waits (each poll is an L2 or memory round
// trip; a wait that is satisfied takes a few microseconds).  After one wait
// of a wave gives up, its later waits give up at once, so a launch whose
// exchanges fail still ends within milliseconds.
constexpr unsigned kXSpinLimit = 1u << 16;

// Pins a value in scalar registers at this point (kernel arguments loaded
// in one batch at the start).
#define ZMOE_PIN(v) asm volatile("" : "+s"(v))

// Whether the workgroups of a G-workgroup launch are dealt to the 8 XCDs in
// turn on the current device (decode1x.hip; scratch: G words of device memory).
bool xcd_round_robin(hipStream_t st, unsigned* scratch, int G);

}  // namespace zmoe
