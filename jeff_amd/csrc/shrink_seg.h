// The LoRA first factor for short segments (decode): the segment form of the shrink (shrink.hip's
// shrink_seg_kernel).
#pragma once

#include "tile_common.h"

namespace mlora {

// The (matrix, 32-rank block) of block index b of an adapter whose live ranks are rk[].
__device__ __forceinline__ void rank_block(const int* rk, int n_mats, int b, int& j, int& kb) {
  j = 0;
  while (j + 1 < n_mats && b >= ((rk[j] + 31) >> 5)) {
    b -= (rk[j] + 31) >> 5;
    ++j;
  }
  kb = b;
}

constexpr int kDWaves = 8;                // waves per workgroup of the segment form, each a share of the inputs
constexpr int kDChunk = 64;               // inputs per staged chunk of A (32 rank rows of 128 bytes)
constexpr int kSegLds = kDWaves * 2 * 32 * kDChunk;  // bf16 elements of LDS: two chunk buffers per wave
static_assert(kDWaves * 16 * kWave * 2 <= kSegLds / 2, "the waves' sums fit the first half of the LDS");

// Short segments (decode): one workgroup per (segment, 32-rank block of a matrix's capacity); blocks past the
// adapter's live rank of that matrix return at once. Its 8 waves split the input dimension into chunks of 64. A wave
// stages each chunk of its 32 rank rows of A in its own two LDS buffers with buffer loads that write LDS directly
// (an instruction covers 8 whole 128-byte rows: every cache line it touches is used whole), one chunk ahead, and
// loads its token rows of x for the chunk into registers (the segment's rows as the second MFMA operand, rows past
// the segment masked to zero); one 32x32x16 MFMA per 16 inputs accumulates a 32-rank x 32-row block. The waves'
// sums are then added in wave order through LDS and rounded once. Segments longer than 32 rows take their rows 32 at
// a time (A is then re-read from L2). The block's bookkeeping is read in two dependent rounds (segment bounds and
// adapter together, then the adapter's rank and the segment's token order) before the A and x loads. `block` is the
// workgroup's index among the (segment, rank block) pairs; `lds_lo` and `lds_hi` are kSegLds / 2 elements of LDS
// each (waves 0-3 stage A in the first, waves 4-7 in the second; the waves' sums use the first). Every thread of the
// workgroup must call it (it synchronises the workgroup).
__device__ __forceinline__ void shrink_seg_block(const mlora_lora_t& L, const mlora_route_t& r,
                                                 const uint16_t* x, int64_t x_stride, int32_t k,
                                                 uint16_t* __restrict__ mid, int32_t max_blocks, int block,
                                                 uint16_t* __restrict__ lds_lo, uint16_t* __restrict__ lds_hi) {
  const int s = block / max_blocks;
  int j = 0, kb = block - s * max_blocks;  // (matrix, 32-rank block) from the capacities
  while (j + 1 < L.n_mats && kb >= (L.cap[j] + 31) >> 5) {
    kb -= (L.cap[j] + 31) >> 5;
    ++j;
  }
  if (kb * 32 >= L.cap[j]) return;
  // s < max_segs, so all four reads are inside their arrays
  const int nseg = *r.num_segs;
  const int a = r.seg_adapter[s];
  const int64_t sb = r.seg_start[s], se = r.seg_start[s + 1];
  if (s >= nseg || a == 0 || se <= sb) return;  // a == 0: the base row, no first factor
  const int lane = threadIdx.x & 63;
  const int rk = live_rank(L, a, j);
  const int32_t tok0 = r.tok_perm[min(sb + (lane & 31), se - 1)];  // the first row block's tokens
  if (kb * 32 >= rk) return;
  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int n = kb * 32 + (lane & 31);  // this lane's rank row
  const uint32_t amask = n < rk ? 0xFFFFFFFFu : 0u;
  // A rows rho_j + 32 kb .. +31 of the adapter through a buffer resource based at the block (rows past the live rank
  // re-read the block's first row). DMA instruction i fills rows 8 i + (lane >> 3): lane l writes LDS slot l & 7 of
  // its row, which holds 16-byte chunk swz_slot(row, l & 7) of the row's 64 inputs.
  const uint16_t* ablk = L.pool + (int64_t)a * L.pool_stride + L.off_a + (int64_t)(rank_offset(L, j) + kb * 32) * k;
  const __amdgpu_buffer_rsrc_t ares =
      __builtin_amdgcn_make_buffer_rsrc((void*)ablk, (short)0, (int)(32 * k * 2), 0x00020000);
  const int live_rows = min(rk - kb * 32, 32);
  uint32_t aoff[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int row = 8 * i + (lane >> 3);
    aoff[i] = (uint32_t)(((row < live_rows ? row : 0) * k + (swz_slot(row, lane & 7) << 3)) * 2);
  }
  uint16_t* buf0 = (wave < kDWaves / 2 ? lds_lo : lds_hi) + (wave % (kDWaves / 2)) * (2 * 32 * kDChunk);
  uint16_t* buf1 = buf0 + 32 * kDChunk;
  auto dma_a = [&](uint16_t* buf, int kc) __attribute__((always_inline)) {
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // this wave's reads of the buffer are done
#pragma unroll
    for (int i = 0; i < 4; ++i)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(ares, (lds_void*)(buf + i * 8 * kDChunk), 16, aoff[i], kc * 2, 0, kReadOnce);
  };
  const int chunks = k / kDChunk;
  const int ch0 = (wave * chunks) / kDWaves, ch1 = ((wave + 1) * chunks) / kDWaves;  // this wave's chunks
  float* red = reinterpret_cast<float*>(lds_lo);  // 8 waves x 16 x 64 floats: kSegLds / 2 elements
  for (int64_t p0 = sb; p0 < se; p0 += 32) {
    const int64_t prow = p0 + (lane & 31);
    const bool rin = prow < se;
    const uint32_t xmask = rin ? 0xFFFFFFFFu : 0u;
    const int32_t tok = p0 == sb ? tok0 : r.tok_perm[rin ? prow : p0];
    const uint16_t* xrow = x + (int64_t)tok * x_stride + 8 * (lane >> 5);
    f32x16_t acc = f32x16_t{};
    auto load_x = [&](uint4 (&xq)[4], int c) __attribute__((always_inline)) {
#pragma unroll
      for (int u = 0; u < 4; ++u) xq[u] = *reinterpret_cast<const uint4*>(xrow + c * kDChunk + 16 * u);
    };
    // chunk c: A operands from its LDS buffer (row = rank lane & 31, 16-byte chunk 2 u + (lane >> 5)), x from xq
    // (zero when `live` is false: a chunk past the wave's last, re-read only to keep the loop free of branches)
    auto compute = [&](const uint16_t* buf, const uint4 (&xq)[4], bool live) __attribute__((always_inline)) {
      const uint4* bv = reinterpret_cast<const uint4*>(buf);
      const uint32_t xm4 = live ? xmask : 0u;
      uint4 av[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) av[u] = bv[swz(lane & 31, 2 * u + (lane >> 5)) >> 3];
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const uint4 am = make_uint4(av[u].x & amask, av[u].y & amask, av[u].z & amask, av[u].w & amask);
        const uint4 xm = make_uint4(xq[u].x & xm4, xq[u].y & xm4, xq[u].z & xm4, xq[u].w & xm4);
        acc = mfma32(am, xm, acc);
      }
    };
    if (ch1 > ch0) {
      // Chunk c + 1's A rows and x are issued before chunk c is used: 8 loads (4 into LDS, 4 into registers) per
      // chunk, so chunk c has landed when at most 8 are outstanding. The count holds only if no load moves across a
      // wait: the loop body has no branch (a chunk past the wave's last is re-read and multiplied by zero), x is not
      // a restrict pointer (so the waits' memory clobbers pin its loads), and scheduling barriers fence the waits.
      uint4 x0[4], x1[4];
      dma_a(buf0, ch0 * kDChunk);
      load_x(x0, ch0);
      for (int c = ch0; c < ch1; c += 2) {
        dma_a(buf1, min(c + 1, ch1 - 1) * kDChunk);
        load_x(x1, min(c + 1, ch1 - 1));
        __builtin_amdgcn_sched_barrier(0);
        asm volatile("s_waitcnt vmcnt(8)" ::: "memory");  // chunk c landed (no LDS read moves above this)
        __builtin_amdgcn_sched_barrier(0);
        compute(buf0, x0, true);
        dma_a(buf0, min(c + 2, ch1 - 1) * kDChunk);
        load_x(x0, min(c + 2, ch1 - 1));
        __builtin_amdgcn_sched_barrier(0);
        asm volatile("s_waitcnt vmcnt(8)" ::: "memory");  // chunk c + 1 landed
        __builtin_amdgcn_sched_barrier(0);
        compute(buf1, x1, c + 1 < ch1);
      }
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // the last re-reads into LDS have landed
    }
    __syncthreads();  // every wave is done with its LDS buffers (and the previous row block's sums are read)
#pragma unroll
    for (int i = 0; i < 16; ++i) red[(wave * 16 + i) * kWave + lane] = acc[i];
    __syncthreads();
    for (int e = tid; e < 16 * kWave; e += kDWaves * kWave) {
      const int i = e / kWave, ln = e % kWave;
      float sum = red[i * kWave + ln];
#pragma unroll
      for (int w = 1; w < kDWaves; ++w) sum += red[(w * 16 + i) * kWave + ln];
      const int q = kb * 32 + (i >> 2) * 8 + (ln >> 5) * 4 + (i & 3);
      const int64_t p = p0 + (ln & 31);
      if (q < rk && p < se) mid[p * L.rank_cap + rank_offset(L, j) + q] = f32_to_bf16(sum);
    }
    __syncthreads();  // the sums are read before the next row block's A chunks overwrite them
  }
}

}  // namespace mlora
