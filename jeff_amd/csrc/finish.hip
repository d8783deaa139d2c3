// Second launch of a split INT4 product (decode-shaped passes: many adapters, few tokens each):
//   y[perm[p], c] = bf16( sum_s part[s][p][c]  +  sum_q mid[p, rho_j + q] sB_j[a][c - o_j, q] )
// part[s] holds the float32 base product of input range s (gemm256.hip, split mode), summed here in range order;
// the LoRA term follows in rank order, in float32, and the sum is rounded once: the reference's epilogue of a split
// product (engine/int4_kernels.py:105-129), with its per-tile adapter replaced by the tile's adapter segment.
//
// One workgroup per (adapter segment, 256 columns of one matrix j), one column per thread. The sB rows of those
// columns are one contiguous block of the pool row (columns x the adapter's sB row stride, bf16), read with coalesced
// 16-byte loads into LDS rows padded by 16 bytes (72 elements: the 16-byte reads of 16 consecutive rows then fall on
// distinct banks); each thread then takes its row from LDS, and the rows' first factors (the same for
// every thread) from LDS as well. A workgroup issues all its loads (partials, sB, first factors) before its first
// barrier, so it waits for memory once; each adapter's sB is read once per pass, and the many small workgroups of
// a pass keep the loads of many segments in flight.
#include "mlora_common.h"

namespace {

using namespace mlora;

constexpr int kFinThreads = 256;  // one output column per thread
constexpr int kFinRows = 8;       // sorted rows per pass
constexpr int kFinRanks = 64;     // sB ranks staged per pass
constexpr int kFinPitch = kFinRanks + 8;
constexpr int kRegRows = 4;     // sorted rows per pass of the register form (decode segments hold a few)
constexpr int kMaxSplit = 8;     // input ranges of a split product (the host picks at most this many)

__global__ __launch_bounds__(kFinThreads) void finish_lds_kernel(mlora_lora_t L, mlora_route_t r,
                                                            const float* __restrict__ part, int32_t ksplit,
                                                            int32_t ld, const uint16_t* __restrict__ mid,
                                                            uint16_t* __restrict__ y, int64_t y_stride,
                                                            uint16_t* __restrict__ last_out, int32_t n_out) {
  __shared__ __attribute__((aligned(16))) uint16_t bs[kFinThreads * kFinPitch];
  __shared__ __attribute__((aligned(16))) uint16_t ms[kFinRows * kFinRanks];
  const int s = blockIdx.y;
  if (s >= *r.num_segs) return;
  const int64_t sb = r.seg_start[s], se = r.seg_start[s + 1];
  if (se <= sb) return;
  // blockIdx.x -> matrix j and its column block
  int j = 0, cb = blockIdx.x, oj = 0;
  while (j + 1 < L.n_mats && cb >= (L.cols[j] + kFinThreads - 1) / kFinThreads) {
    cb -= (L.cols[j] + kFinThreads - 1) / kFinThreads;
    oj += L.cols[j];
    ++j;
  }
  const int c0 = cb * kFinThreads;  // first column of the block within matrix j
  const int ncols = min(kFinThreads, L.cols[j] - c0);
  if (ncols <= 0) return;
  const int tid = threadIdx.x;
  const bool cok = tid < ncols;
  const int c = oj + c0 + tid;  // output column
  const int a = r.seg_adapter[s];
  const int rk = a != 0 ? live_rank(L, a, j) : 0;
  const int sbs = sb_stride(rk, L.cap[j]);  // the adapter's sB row stride
  const int rho = rank_offset(L, j);
  const int rc = L.rank_cap;
  const uint16_t* blk = L.pool + (int64_t)a * L.pool_stride + L.off_b[j] + (int64_t)c0 * sbs;
  const int64_t T = r.tokens;
  for (int64_t p0 = sb; p0 < se; p0 += kFinRows) {
    const int rows = (int)min((int64_t)kFinRows, se - p0);
    // Every load of the pass is issued before the first use: the partial sums of the thread's column, its sB row
    // chunks (registers, then LDS) and the rows' first factors (LDS).
    float pv[kMaxSplit][kFinRows];
#pragma unroll
    for (int sp = 0; sp < kMaxSplit; ++sp)
#pragma unroll
      for (int rr = 0; rr < kFinRows; ++rr)
        pv[sp][rr] = (cok && sp < ksplit && rr < rows) ? part[((int64_t)sp * T + p0 + rr) * ld + c] : 0.0f;
    for (int q0 = 0; q0 < max(rk, 1); q0 += kFinRanks) {
      const int nq = min(rk - q0, kFinRanks);  // live ranks of this chunk (none for the base row)
      const int chunks = min(kFinRanks, sbs - q0) / 8;
      uint4 bv[kFinRanks / 8];
#pragma unroll
      for (int i = 0; i < kFinRanks / 8; ++i) {
        const int e = tid + kFinThreads * i;
        const int col = e / max(chunks, 1), ch = e - col * max(chunks, 1);
        bv[i] = (nq > 0 && col < ncols) ? *reinterpret_cast<const uint4*>(blk + (int64_t)col * sbs + q0 + 8 * ch)
                                        : make_uint4(0, 0, 0, 0);
      }
      const int mrow = tid / (kFinRanks / 8), mch = tid % (kFinRanks / 8);
      const uint4 mv = (nq > 0 && mrow < rows && 8 * mch < nq)
                           ? *reinterpret_cast<const uint4*>(mid + (p0 + mrow) * rc + rho + q0 + 8 * mch)
                           : make_uint4(0, 0, 0, 0);
      __syncthreads();  // the previous chunk's readers are done with bs and ms
#pragma unroll
      for (int i = 0; i < kFinRanks / 8; ++i) {
        const int e = tid + kFinThreads * i;
        const int col = e / max(chunks, 1), ch = e - col * max(chunks, 1);
        if (nq > 0 && col < ncols) *reinterpret_cast<uint4*>(&bs[col * kFinPitch + 8 * ch]) = bv[i];
      }
      if (mrow < kFinRows) *reinterpret_cast<uint4*>(&ms[mrow * kFinRanks + 8 * mch]) = mv;
      __syncthreads();
      if (q0 == 0) {  // the base partial sums first, in range order
#pragma unroll
        for (int rr = 0; rr < kFinRows; ++rr) {
          float v = 0.0f;
#pragma unroll
          for (int sp = 0; sp < kMaxSplit; ++sp) v += pv[sp][rr];
          pv[0][rr] = v;
        }
      }
      if (cok) {
        for (int i = 0; i < (nq + 7) / 8; ++i) {
          // ranks past the live rank are skipped, not multiplied by zero: the first factors there are not written
          const int n8 = min(8, nq - 8 * i);
          const uint4 b4 = *reinterpret_cast<const uint4*>(&bs[tid * kFinPitch + 8 * i]);
          const uint32_t bw[4] = {b4.x, b4.y, b4.z, b4.w};
#pragma unroll
          for (int rr = 0; rr < kFinRows; ++rr) {
            if (rr >= rows) break;
            const uint4 m4 = *reinterpret_cast<const uint4*>(&ms[rr * kFinRanks + 8 * i]);
            const uint32_t mw[4] = {m4.x, m4.y, m4.z, m4.w};
#pragma unroll
            for (int e = 0; e < 8; ++e) {
              if (e >= n8) break;
              const float bf = bf16_to_f32((bw[e >> 1] >> (16 * (e & 1))) & 0xFFFFu);
              const float mf = bf16_to_f32((mw[e >> 1] >> (16 * (e & 1))) & 0xFFFFu);
              pv[0][rr] = __builtin_fmaf(mf, bf, pv[0][rr]);
            }
          }
        }
      }
    }
    if (!cok) continue;
#pragma unroll
    for (int rr = 0; rr < kFinRows; ++rr) {
      if (rr >= rows) break;
      const int64_t p = p0 + rr;
      const uint16_t v = f32_to_bf16(pv[0][rr]);
      y[(int64_t)r.tok_perm[p] * y_stride + c] = v;
      if (last_out != nullptr) {
        const int q = r.last_of[p];
        if (q >= 0) last_out[(int64_t)q * n_out + c] = v;
      }
    }
  }
}

// Sum of v over the CPC consecutive lanes of a column group (CPC = 1, 2, 4 or 8), every lane of the group ending with
// the same bits: DPP lane moves (xor 1, xor 2 within quads, then the mirrored quad of the 8-lane half row), each
// step adding two equal-order partial sums.
template <int CPC>
__device__ __forceinline__ float group_sum(float v) {
  if constexpr (CPC >= 2)
    v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0xB1, 0xF, 0xF, false));
  if constexpr (CPC >= 4)
    v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x4E, 0xF, 0xF, false));
  if constexpr (CPC >= 8)
    v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x141, 0xF, 0xF, false));
  return v;
}

// One (segment, 256 columns of matrix j) of an adapter whose sB rows hold CPC * 8 ranks (row stride 8, 16, 32 or 64).
// Thread t takes 16-byte chunk t % CPC of the rows of columns t / CPC + (256 / CPC) i, i < CPC: consecutive threads
// read consecutive 16 bytes of the contiguous sB block. Per pass of kRegRows rows:
//  - every thread sums four columns of one row's base partials over the input ranges (coalesced 16-byte loads, all
//    ranges in flight) into LDS;
//  - each lane dots its sB chunk with the same ranks of every row's first factor, the CPC lanes of a column add
//    their partial sums (group_sum), and lane t % CPC == row % CPC adds the base sum and rounds into an LDS tile;
//  - the tile's rows are written with coalesced 8-byte stores.
template <int CPC, int MAXS>
__device__ __forceinline__ void finish_columns(const mlora_lora_t& L, const mlora_route_t& r,
                                               const float* __restrict__ part, int32_t ksplit, int32_t ld,
                                               const uint16_t* __restrict__ mid, uint16_t* __restrict__ y,
                                               int64_t y_stride, uint16_t* __restrict__ last_out, int32_t n_out,
                                               int64_t sb, int64_t se, int a, int j, int oj, int c0, int ncols,
                                               int32_t vec, float* __restrict__ base_lds,
                                               uint16_t* __restrict__ out_lds) {
  const int tid = threadIdx.x;
  const int ch = tid % CPC, cl = tid / CPC;
  const int rk = a != 0 ? live_rank(L, a, j) : 0;
  const int rho = rank_offset(L, j);
  const int rc = L.rank_cap;
  const bool chunk_live = 8 * ch < rk;
  const uint16_t* blk = L.pool + (int64_t)a * L.pool_stride + L.off_b[j] + (int64_t)c0 * (8 * CPC);
  const int64_t T = r.tokens;
  uint4 bv[CPC];
  // the thread's four columns of one row for the base sums and the stores
  const int srow = tid / (kFinThreads / 4), scol = 4 * (tid % (kFinThreads / 4));
  for (int64_t p0 = sb; p0 < se; p0 += kRegRows) {
    const int rows = (int)min((int64_t)kRegRows, se - p0);
    // where the thread's row goes, fetched before anything that waits
    const int64_t prow = p0 + min(srow, rows - 1);
    const int64_t yrow_off = (int64_t)r.tok_perm[prow] * y_stride;
    const int q = last_out != nullptr ? r.last_of[prow] : -1;
    // base partial sums, in range order
    float4 pv[MAXS];
#pragma unroll
    for (int sp = 0; sp < MAXS; ++sp)
      pv[sp] = (sp < ksplit && srow < rows && scol < ncols)
                   ? *reinterpret_cast<const float4*>(part + ((int64_t)sp * T + p0 + srow) * ld + oj + c0 + scol)
                   : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    // first factors of the rows, this lane's 8 ranks; ranks past the live rank masked to zero (they are not written)
    uint4 mv[kRegRows];
#pragma unroll
    for (int rr = 0; rr < kRegRows; ++rr)
      mv[rr] = (chunk_live && rr < rows)
                   ? keep_first(*reinterpret_cast<const uint4*>(mid + (p0 + rr) * rc + rho + 8 * ch), rk - 8 * ch)
                   : make_uint4(0, 0, 0, 0);
    if (p0 == sb) {  // the block's sB rows, issued after the first pass's partial sums (needed first)
#pragma unroll
      for (int i = 0; i < CPC; ++i) {
        const int col = cl + (kFinThreads / CPC) * i;
        bv[i] = (chunk_live && col < ncols)
                    ? keep_first(*reinterpret_cast<const uint4*>(blk + (int64_t)col * (8 * CPC) + 8 * ch), rk - 8 * ch)
                    : make_uint4(0, 0, 0, 0);
      }
    }
    float4 bsum = pv[0];
#pragma unroll
    for (int sp = 1; sp < MAXS; ++sp) {
      bsum.x += pv[sp].x;
      bsum.y += pv[sp].y;
      bsum.z += pv[sp].z;
      bsum.w += pv[sp].w;
    }
    __syncthreads();  // the previous pass is done with both LDS tiles
    *reinterpret_cast<float4*>(&base_lds[srow * kFinThreads + scol]) = bsum;
    __syncthreads();
#pragma unroll
    for (int i = 0; i < CPC; ++i) {
      const int col = cl + (kFinThreads / CPC) * i;
#pragma unroll
      for (int rr = 0; rr < kRegRows; ++rr) {
        if (rr >= rows) break;
        const float lora = group_sum<CPC>(dot8(bv[i], mv[rr], 0.0f));
        if (rr % CPC == ch) out_lds[rr * kFinThreads + col] = f32_to_bf16(base_lds[rr * kFinThreads + col] + lora);
      }
    }
    __syncthreads();
    if (srow < rows && scol < ncols) {
      const int c = oj + c0 + scol;
      const uint2 v = *reinterpret_cast<const uint2*>(&out_lds[srow * kFinThreads + scol]);
      store4(y + yrow_off + c, q >= 0 ? last_out + (int64_t)q * n_out + c : nullptr, v.x, v.y, ncols - scol, vec);
    }
  }
}

// The register form of the split product's second launch: every matrix of the group has cap_j in {0, 8, 16, 32, 64}
// (so every adapter's sB row stride is 8, 16, 32 or 64).
// MAXS: the most input ranges this form reads (1 when the base ran as one range, which frees their registers)
template <int MAXS>
__global__ __launch_bounds__(kFinThreads) void finish_kernel(mlora_lora_t L, mlora_route_t r,
                                                            const float* __restrict__ part, int32_t ksplit,
                                                            int32_t ld, const uint16_t* __restrict__ mid,
                                                            uint16_t* __restrict__ y, int64_t y_stride,
                                                            uint16_t* __restrict__ last_out, int32_t n_out,
                                                            int32_t vec) {
  __shared__ __attribute__((aligned(16))) float base_lds[kRegRows * kFinThreads];
  __shared__ __attribute__((aligned(16))) uint16_t out_lds[kRegRows * kFinThreads];
  const int s = blockIdx.y;
  if (s >= *r.num_segs) return;
  const int64_t sb = r.seg_start[s], se = r.seg_start[s + 1];
  if (se <= sb) return;
  int j = 0, cb = blockIdx.x, oj = 0;
  while (j + 1 < L.n_mats && cb >= (L.cols[j] + kFinThreads - 1) / kFinThreads) {
    cb -= (L.cols[j] + kFinThreads - 1) / kFinThreads;
    oj += L.cols[j];
    ++j;
  }
  const int c0 = cb * kFinThreads;
  const int ncols = min(kFinThreads, L.cols[j] - c0);
  if (ncols <= 0) return;
  const int a = r.seg_adapter[s];
  switch (sb_stride(a != 0 ? live_rank(L, a, j) : 0, L.cap[j])) {  // the adapter's sB row stride
    case 64:
      finish_columns<8, MAXS>(L, r, part, ksplit, ld, mid, y, y_stride, last_out, n_out, sb, se, a, j, oj, c0, ncols,
                        vec, base_lds, out_lds);
      break;
    case 32:
      finish_columns<4, MAXS>(L, r, part, ksplit, ld, mid, y, y_stride, last_out, n_out, sb, se, a, j, oj, c0, ncols,
                        vec, base_lds, out_lds);
      break;
    case 16:
      finish_columns<2, MAXS>(L, r, part, ksplit, ld, mid, y, y_stride, last_out, n_out, sb, se, a, j, oj, c0, ncols,
                        vec, base_lds, out_lds);
      break;
    default:  // 8, or 0 (no adapter on this matrix: the base partial sums only)
      finish_columns<1, MAXS>(L, r, part, ksplit, ld, mid, y, y_stride, last_out, n_out, sb, se, a, j, oj, c0, ncols,
                        vec, base_lds, out_lds);
      break;
  }
}

// The gated form (the group's matrices 0 and 1 are gate and up, inter columns each): one workgroup per (segment, 128
// output columns c0 .. c0 + 127); threads 0..127 finish gate columns c0 .. +127 and threads 128..255 the same up
// columns, each half as finish_columns does with 128 threads (CPC chunks per column, CPC from the larger of the two
// sB row strides: the half with the smaller stride leaves the extra chunks unread and zero). The gate half then pairs
// its rounded outputs with the up half's in LDS and writes silu(gate) * up.
template <int CPC, int MAXS>
__device__ __forceinline__ void finish_gated_columns(const mlora_lora_t& L, const mlora_route_t& r,
                                                     const float* __restrict__ part, int32_t ksplit, int32_t ld,
                                                     const uint16_t* __restrict__ mid, uint16_t* __restrict__ y,
                                                     int64_t y_stride, uint16_t* __restrict__ last_out, int32_t inter,
                                                     int64_t sb, int64_t se, int a, int c0, bool vec,
                                                     float* __restrict__ base_lds, uint16_t* __restrict__ out_lds) {
  const int tid = threadIdx.x;
  const int h = tid >> 7, t = tid & 127;  // half (matrix j = h) and thread within it
  const int ch = t % CPC, cl = t / CPC;
  const int rk = a != 0 ? live_rank(L, a, h) : 0;
  const int rho = rank_offset(L, h);
  const int rc = L.rank_cap;
  const int sbs = sb_stride(rk, L.cap[h]);
  const bool chunk_live = 8 * ch < rk;
  const uint16_t* blk = L.pool + (int64_t)a * L.pool_stride + L.off_b[h] + (int64_t)c0 * sbs;
  const int64_t T = r.tokens;
  const int oj = h * inter;  // the half's first column in the group's output order
  uint4 bv[CPC];
  const int srow = t / 32, scol = 4 * (t % 32);
  for (int64_t p0 = sb; p0 < se; p0 += kRegRows) {
    const int rows = (int)min((int64_t)kRegRows, se - p0);
    const int64_t prow = p0 + min(srow, rows - 1);
    const int64_t yrow_off = (int64_t)r.tok_perm[prow] * y_stride;
    const int q = last_out != nullptr ? r.last_of[prow] : -1;
    float4 pv[MAXS];
#pragma unroll
    for (int sp = 0; sp < MAXS; ++sp)
      pv[sp] = (sp < ksplit && srow < rows)
                   ? *reinterpret_cast<const float4*>(part + ((int64_t)sp * T + p0 + srow) * ld + oj + c0 + scol)
                   : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    uint4 mv[kRegRows];
#pragma unroll
    for (int rr = 0; rr < kRegRows; ++rr)
      mv[rr] = (chunk_live && rr < rows)
                   ? keep_first(*reinterpret_cast<const uint4*>(mid + (p0 + rr) * rc + rho + 8 * ch), rk - 8 * ch)
                   : make_uint4(0, 0, 0, 0);
    if (p0 == sb) {
#pragma unroll
      for (int i = 0; i < CPC; ++i) {
        const int col = cl + (128 / CPC) * i;
        bv[i] = chunk_live ? keep_first(*reinterpret_cast<const uint4*>(blk + (int64_t)col * sbs + 8 * ch), rk - 8 * ch)
                           : make_uint4(0, 0, 0, 0);
      }
    }
    float4 bsum = pv[0];
#pragma unroll
    for (int sp = 1; sp < MAXS; ++sp) {
      bsum.x += pv[sp].x;
      bsum.y += pv[sp].y;
      bsum.z += pv[sp].z;
      bsum.w += pv[sp].w;
    }
    __syncthreads();  // the previous pass is done with both LDS tiles
    *reinterpret_cast<float4*>(&base_lds[srow * kFinThreads + h * 128 + scol]) = bsum;
    __syncthreads();
#pragma unroll
    for (int i = 0; i < CPC; ++i) {
      const int col = h * 128 + cl + (128 / CPC) * i;
#pragma unroll
      for (int rr = 0; rr < kRegRows; ++rr) {
        if (rr >= rows) break;
        const float lora = group_sum<CPC>(dot8(bv[i], mv[rr], 0.0f));
        if (rr % CPC == ch) out_lds[rr * kFinThreads + col] = f32_to_bf16(base_lds[rr * kFinThreads + col] + lora);
      }
    }
    __syncthreads();
    if (h == 0 && srow < rows) {
      const uint2 g = *reinterpret_cast<const uint2*>(&out_lds[srow * kFinThreads + scol]);
      const uint2 u = *reinterpret_cast<const uint2*>(&out_lds[srow * kFinThreads + 128 + scol]);
      const uint2 v = silu_mul4(g, u);
      // (the column offset is opaque so the output addresses are formed here: hoisted out of the row loop, the
      // last-token row's 64-bit address did not fit the registers and went to scratch memory, once per thread)
      int c = c0 + scol;
      asm volatile("" : "+v"(c));
      uint16_t* yrow = y + yrow_off;
      if (vec) {
        *reinterpret_cast<uint2*>(yrow + c) = v;
        if (q >= 0) *reinterpret_cast<uint2*>(last_out + (int64_t)q * inter + c) = v;
      } else {
        const uint16_t hv[4] = {(uint16_t)v.x, (uint16_t)(v.x >> 16), (uint16_t)v.y, (uint16_t)(v.y >> 16)};
        for (int e = 0; e < 4; ++e) {
          yrow[c + e] = hv[e];
          if (q >= 0) last_out[(int64_t)q * inter + c + e] = hv[e];
        }
      }
    }
  }
}

// (one input range: five waves per SIMD, as the plain form's 91 registers allow, so the loads of more segments are
// in flight)
template <int MAXS>
__global__ __launch_bounds__(kFinThreads) __attribute__((amdgpu_waves_per_eu(MAXS == 1 ? 5 : 3))) void
finish_gated_kernel(mlora_lora_t L, mlora_route_t r,
                                                                  const float* __restrict__ part, int32_t ksplit,
                                                                  int32_t ld, const uint16_t* __restrict__ mid,
                                                                  uint16_t* __restrict__ y, int64_t y_stride,
                                                                  uint16_t* __restrict__ last_out, int32_t inter,
                                                                  int32_t vec) {
  __shared__ __attribute__((aligned(16))) float base_lds[kRegRows * kFinThreads];
  __shared__ __attribute__((aligned(16))) uint16_t out_lds[kRegRows * kFinThreads];
  const int s = blockIdx.y;
  if (s >= *r.num_segs) return;
  const int64_t sb = r.seg_start[s], se = r.seg_start[s + 1];
  if (se <= sb) return;
  const int c0 = blockIdx.x * 128;
  const int a = r.seg_adapter[s];
  const int sg = sb_stride(a != 0 ? live_rank(L, a, 0) : 0, L.cap[0]);
  const int su = sb_stride(a != 0 ? live_rank(L, a, 1) : 0, L.cap[1]);
  switch (max(sg, su)) {  // the larger sB row stride of the two matrices
    case 64:
      finish_gated_columns<8, MAXS>(L, r, part, ksplit, ld, mid, y, y_stride, last_out, inter, sb, se, a, c0,
                                    vec, base_lds, out_lds);
      break;
    case 32:
      finish_gated_columns<4, MAXS>(L, r, part, ksplit, ld, mid, y, y_stride, last_out, inter, sb, se, a, c0,
                                    vec, base_lds, out_lds);
      break;
    case 16:
      finish_gated_columns<2, MAXS>(L, r, part, ksplit, ld, mid, y, y_stride, last_out, inter, sb, se, a, c0,
                                    vec, base_lds, out_lds);
      break;
    default:
      finish_gated_columns<1, MAXS>(L, r, part, ksplit, ld, mid, y, y_stride, last_out, inter, sb, se, a, c0,
                                    vec, base_lds, out_lds);
      break;
  }
}

}  // namespace

bool finish_registers(const mlora_lora_t& L) {
  bool ok = true;
  for (int j = 0; j < L.n_mats; ++j) {
    const int c = L.cap[j];
    ok = ok && (c == 0 || c == 8 || c == 16 || c == 32 || c == 64) && L.cols[j] % 4 == 0;
  }
  return ok;
}

int launch_finish(const mlora_lora_t& L, const mlora_route_t& r, const float* part, int32_t ksplit, int32_t ld,
                  const uint16_t* mid, uint16_t* y, int64_t y_stride, uint16_t* last_out, int32_t n_out,
                  hipStream_t stream, int32_t inter, bool residual) {
  if (r.tokens == 0 || n_out == 0 || r.max_segs == 0) return MLORA_OK;
  if (inter > 0) {
    if (residual) return MLORA_EINVAL;
    if (inter % 128 || L.n_mats != 2 || L.cols[0] != inter || L.cols[1] != inter || !finish_registers(L))
      return MLORA_EINVAL;
    const dim3 grid((unsigned)(inter / 128), (unsigned)r.max_segs);
    const bool vec = reinterpret_cast<uintptr_t>(y) % 8 == 0 && y_stride % 4 == 0 &&
                     (last_out == nullptr || reinterpret_cast<uintptr_t>(last_out) % 8 == 0);
    if (ksplit == 1)
      hipLaunchKernelGGL(finish_gated_kernel<1>, grid, dim3(kFinThreads), 0, stream, L, r, part, ksplit, ld, mid, y,
                         y_stride, last_out, inter, (int32_t)vec);
    else
      hipLaunchKernelGGL(finish_gated_kernel<kMaxSplit>, grid, dim3(kFinThreads), 0, stream, L, r, part, ksplit, ld,
                         mid, y, y_stride, last_out, inter, (int32_t)vec);
    return hipGetLastError() == hipSuccess ? MLORA_OK : MLORA_ELAUNCH;
  }
  int blocks = 0;
  // the register form: every cap_j in {0, 8, 16, 32, 64} and every matrix a multiple of four columns (its partial
  // sums are read four columns at a time)
  const bool registers = finish_registers(L);
  if (residual && !registers) return MLORA_EINVAL;
  for (int j = 0; j < L.n_mats; ++j) blocks += (L.cols[j] + kFinThreads - 1) / kFinThreads;
  const dim3 grid((unsigned)blocks, (unsigned)r.max_segs);
  // 8-byte stores of four columns: 8-byte aligned output rows
  const int32_t vec = (reinterpret_cast<uintptr_t>(y) % 8 == 0 && y_stride % 4 == 0 &&
                               (last_out == nullptr ||
                                (reinterpret_cast<uintptr_t>(last_out) % 8 == 0 && n_out % 4 == 0))
                           ? kStoreVec
                           : 0) |
                      (residual ? kStoreResidual : 0);
  if (registers && ksplit == 1)
    hipLaunchKernelGGL(finish_kernel<1>, grid, dim3(kFinThreads), 0, stream, L, r, part, ksplit, ld, mid, y, y_stride,
                       last_out, n_out, vec);
  else if (registers)
    hipLaunchKernelGGL(finish_kernel<kMaxSplit>, grid, dim3(kFinThreads), 0, stream, L, r, part, ksplit, ld, mid, y,
                       y_stride, last_out, n_out, vec);
  else
    hipLaunchKernelGGL(finish_lds_kernel, grid, dim3(kFinThreads), 0, stream, L, r, part, ksplit, ld, mid, y,
                       y_stride, last_out, n_out);
  return hipGetLastError() == hipSuccess ? MLORA_OK : MLORA_ELAUNCH;
}
