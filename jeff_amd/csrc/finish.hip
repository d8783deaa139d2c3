// Second launch of a split INT4 product (decode-shaped passes: many adapters, few tokens each):
//   y[perm[p], c] = bf16( sum_s part[s][p][c]  +  sum_q mid[p, rho_j + q] sB_j[a][c - o_j, q] )
// part[s] holds the float32 base product of input range s (gemm256.hip, split mode), summed here in range order;
// the LoRA term follows in rank order, in float32, and the sum is rounded once: the reference's epilogue of a split
// product (engine/int4_kernels.py:105-129), with its per-tile adapter replaced by the tile's adapter segment.
//
// One workgroup per (adapter segment, 256 columns of one matrix j), one column per thread. The sB rows of those
// columns are one contiguous block of the pool row (columns x cap_j bf16), read with coalesced 16-byte loads into
// LDS rows padded by 16 bytes (cap_j + 8 elements: the 16-byte reads of 16 consecutive rows then fall on distinct
// banks when cap_j / 8 is even); each thread then takes its row from LDS, and the rows' first factors (the same for
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
constexpr int kMaxSplit = 8;     // input ranges of a split product (the host picks at most this many)

__global__ __launch_bounds__(kFinThreads) void finish_kernel(mlora_lora_t L, mlora_route_t r,
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
  const int capj = L.cap[j];
  const int rk = a != 0 ? live_rank(L, a, j) : 0;
  const int rho = rank_offset(L, j);
  const int rc = L.rank_cap;
  const uint16_t* blk = L.pool + (int64_t)a * L.pool_stride + L.off_b[j] + (int64_t)c0 * capj;
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
      const int chunks = min(kFinRanks, capj - q0) / 8;
      uint4 bv[kFinRanks / 8];
#pragma unroll
      for (int i = 0; i < kFinRanks / 8; ++i) {
        const int e = tid + kFinThreads * i;
        const int col = e / max(chunks, 1), ch = e - col * max(chunks, 1);
        bv[i] = (nq > 0 && col < ncols) ? *reinterpret_cast<const uint4*>(blk + (int64_t)col * capj + q0 + 8 * ch)
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

}  // namespace

int launch_finish(const mlora_lora_t& L, const mlora_route_t& r, const float* part, int32_t ksplit, int32_t ld,
                  const uint16_t* mid, uint16_t* y, int64_t y_stride, uint16_t* last_out, int32_t n_out,
                  hipStream_t stream) {
  if (r.tokens == 0 || n_out == 0 || r.max_segs == 0) return MLORA_OK;
  int blocks = 0;
  for (int j = 0; j < L.n_mats; ++j) blocks += (L.cols[j] + kFinThreads - 1) / kFinThreads;
  const dim3 grid((unsigned)blocks, (unsigned)r.max_segs);
  hipLaunchKernelGGL(finish_kernel, grid, dim3(kFinThreads), 0, stream, L, r, part, ksplit, ld, mid, y, y_stride,
                     last_out, n_out);
  return hipGetLastError() == hipSuccess ? MLORA_OK : MLORA_ELAUNCH;
}
