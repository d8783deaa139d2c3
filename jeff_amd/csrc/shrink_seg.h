// The LoRA first factor for short segments (decode), shared by its own kernel (shrink.hip) and by the split
// product's first launch (gemm256.hip), whose extra workgroups compute it beside the base product's ranges.
#pragma once

#include "mlora_common.h"

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

constexpr int kDWaves = 8;   // waves per workgroup of the segment form, each a contiguous share of the inputs
constexpr int kDUnroll = 4;  // 16-input steps per load batch; two batches in flight (two workgroups per CU)

// Short segments (decode): one workgroup per (segment, 32-rank block of a matrix's capacity); blocks past the
// adapter's live rank of that matrix return at once. Its 8 waves split the input dimension; a lane streams its rank
// row of A and its token row of x (the segment's rows as the second MFMA operand, rows past the segment masked to
// zero) straight into MFMA operands, 8 steps of 16 inputs in flight; one 32x32x16 MFMA per step accumulates a
// 32-rank x 32-row block. The waves' sums are added in wave order through LDS and rounded once. Segments longer than
// 32 rows take their rows 32 at a time (A is then re-read from L2). The block's bookkeeping is read in two dependent
// rounds (segment bounds and adapter together, then the adapter's rank and the segment's token order) before the
// A and x loads. `block` is the workgroup's index among the (segment, rank block) pairs, `red` 32 KB of LDS. Every
// thread of the workgroup must call it (it synchronises the workgroup).
__device__ __forceinline__ void shrink_seg_block(const mlora_lora_t& L, const mlora_route_t& r,
                                                 const uint16_t* __restrict__ x, int64_t x_stride, int32_t k,
                                                 uint16_t* __restrict__ mid, int32_t max_blocks, int block,
                                                 float* __restrict__ red) {
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
  const int tid = threadIdx.x, wave = tid >> 6;
  const int n = kb * 32 + (lane & 31);  // this lane's rank row
  const bool aok = n < rk;
  const uint32_t amask = aok ? 0xFFFFFFFFu : 0u;
  const uint16_t* arow =
      L.pool + (int64_t)a * L.pool_stride + L.off_a + (int64_t)(rank_offset(L, j) + (aok ? n : 0)) * k + 8 * (lane >> 5);
  const int steps = k / 16;
  const int c0 = (wave * steps) / kDWaves, c1 = ((wave + 1) * steps) / kDWaves;  // this wave's 16-input steps
  for (int64_t p0 = sb; p0 < se; p0 += 32) {
    const int64_t prow = p0 + (lane & 31);
    const bool rin = prow < se;
    const uint32_t xmask = rin ? 0xFFFFFFFFu : 0u;
    const int32_t tok = p0 == sb ? tok0 : r.tok_perm[rin ? prow : p0];
    const uint16_t* xrow = x + (int64_t)tok * x_stride + 8 * (lane >> 5);
    f32x16_t acc = f32x16_t{};
    // every load is unconditional (steps past the wave's range re-read its last one and are not multiplied)
    uint4 av[2][kDUnroll], xv[2][kDUnroll];
    auto issue = [&](uint4 (&aq)[kDUnroll], uint4 (&xq)[kDUnroll], int c) __attribute__((always_inline)) {
#pragma unroll
      for (int u = 0; u < kDUnroll; ++u) {
        const int kk = max(min(c + u, c1 - 1), c0) * 16;
        aq[u] = *reinterpret_cast<const uint4*>(arow + kk);
        xq[u] = *reinterpret_cast<const uint4*>(xrow + kk);
      }
    };
    auto compute = [&](const uint4 (&aq)[kDUnroll], const uint4 (&xq)[kDUnroll], int c) __attribute__((always_inline)) {
#pragma unroll
      for (int u = 0; u < kDUnroll; ++u) {
        if (c + u >= c1) break;
        const uint4 am = make_uint4(aq[u].x & amask, aq[u].y & amask, aq[u].z & amask, aq[u].w & amask);
        const uint4 xm = make_uint4(xq[u].x & xmask, xq[u].y & xmask, xq[u].z & xmask, xq[u].w & xmask);
        acc = mfma32(am, xm, acc);
      }
    };
    if (c1 > c0) {
      issue(av[0], xv[0], c0);
      for (int c = c0; c < c1; c += 2 * kDUnroll) {
        issue(av[1], xv[1], c + kDUnroll);
        compute(av[0], xv[0], c);
        if (c + kDUnroll >= c1) break;
        issue(av[0], xv[0], c + 2 * kDUnroll);
        compute(av[1], xv[1], c + kDUnroll);
      }
    }
    __syncthreads();  // the previous row block's sums are read
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
  }
}

}  // namespace mlora
