// Pieces shared by the MFMA tile kernels that stage x in LDS (gemm256.hip, decode.hip, shrink.hip): the swizzled
// 64-input LDS row layout, the explicit memory waits and barriers of their K loops, the XCD-aware block order and a
// lane's per-step weight registers.
#pragma once

#include "mlora_common.h"

namespace mlora {

constexpr int kTK = 64;  // inputs per K step (one 128-byte LDS row of bf16)

typedef __attribute__((address_space(3))) void lds_void;

// Swizzled 64-element (128-byte) LDS rows. gfx950's LDS has 64 four-byte banks, so rows 2m and 2m + 1 share one
// 256-byte bank line, and a 16-byte read serves 16 lanes per cycle: the eight 16-byte chunks of a row are
// XOR-permuted by (row >> 1) & 7, so the reads of 16 consecutive rows at one logical chunk hit all 64 banks once.
// swz_slot is the slot holding logical chunk c of row `row` (and, the XOR being its own inverse, the logical chunk
// held in slot c); swz is the element offset of logical chunk c.
__device__ __forceinline__ int swz_slot(int row, int c) { return c ^ ((row >> 1) & 7); }
__device__ __forceinline__ int swz(int row, int c) { return row * kTK + (swz_slot(row, c) << 3); }

// Wait until at most n vector memory instructions of this wave are outstanding and its LDS operations are done
// (gfx9 s_waitcnt encoding: vmcnt in bits 3:0 and 15:14, expcnt 6:4 left at its maximum, lgkmcnt 11:8 = 0).
#define MLORA_WAIT_VM(n) __builtin_amdgcn_s_waitcnt(((n) & 0xF) | (((n) >> 4) << 14) | (0x7 << 4))
// ... and until its LDS operations are done, vector memory instructions left in flight (vmcnt at its maximum, 63)
#define MLORA_WAIT_LGKM0() __builtin_amdgcn_s_waitcnt(0xF | (0x3 << 14) | (0x7 << 4))

// Cache policy of the direct-to-LDS loads of data read once per product (the adapters' sB rows and first-factor A
// rows): the non-temporal bit, so the stream does not push the x rows and weights that other tiles re-read out of
// the caches (decode-pool-28l's step 32.8 -> 32.0 ms).
constexpr int kReadOnce = 2;

// Workgroup barrier that orders LDS accesses only (global stores in flight are not waited for).
__device__ __forceinline__ void lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// Step barrier of a K loop where LDS is written only by the x loads and only read by the waves. The wave's own x
// loads of the next step have landed (MLORA_WAIT_VM before this); its LDS reads are drained inside the asm
// statement, so none can be scheduled between the drain and the barrier; then the barrier. There is no release fence:
// a fence would also wait for the x loads in flight for two steps ahead. The memory clobbers keep the compiler from
// moving LDS reads or loads across the barrier.
__device__ __forceinline__ void step_sync() {
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// blockIdx -> tile index such that consecutive tiles share an XCD (blocks are dealt to the 8 XCDs round-robin)
__device__ __forceinline__ int xcd_tile(int b, int nb) {
  const int per = nb / 8, extra = nb % 8;
  const int xcd = b % 8, slot = b / 8;
  return xcd * per + min(xcd, extra) + slot;
}

// One step's weights as loaded by a lane: word [k16] of its column, and the raw bf16 scale and zero point of its
// column (converted only when used, a step later)
struct WStage {
  uint32_t w[4];
  uint32_t sbits, zbyte;
};

}  // namespace mlora
