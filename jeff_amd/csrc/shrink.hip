// The LoRA first factor ("shrink"): mid[p, rho_j + q] = bf16( sum_k x[perm[p], k] A_j[a][q, k] ) for every sorted
// token position p of an adapter segment, matrix j of the group and live rank q. Summed in float32 in a fixed
// order and rounded once to bf16, as the reference rounds its first factor before the second product
// (engine/fast_path.py:159-177,196; engine/int4_kernels.py:67-82,120). Two kernels, chosen by segment length:
//  - shrink_gemv: few tokens per adapter (decode). One workgroup per (segment, matrix, 16 ranks) streams those 16
//    rows of A once, coalesced, and reduces across the workgroup in a fixed order. Memory-bound on A.
//  - shrink_mfma: long segments (prefill). One workgroup per 64 sorted positions stages x through LDS and runs
//    32x32x16 bf16 MFMAs against each overlapping segment's A.
#include "mlora_common.h"

namespace {

using namespace mlora;

constexpr int kGemvThreads = 256;
constexpr int kGemvRows = 4;    // tokens per pass over A
constexpr int kGemvRanks = 16;  // rank rows of A per workgroup

__global__ __launch_bounds__(kGemvThreads) void shrink_gemv_kernel(mlora_lora_t L, mlora_route_t r,
                                                                  const uint16_t* __restrict__ x, int64_t x_stride,
                                                                  int32_t k, uint16_t* __restrict__ mid,
                                                                  int32_t qchunks) {
  __shared__ float red[kGemvThreads / kWave][kWave];
  const int per_seg = L.n_mats * qchunks;
  const int s = blockIdx.x / per_seg;
  const int rem = blockIdx.x - s * per_seg;
  const int j = rem / qchunks, qc = rem - j * qchunks;
  if (s >= *r.num_segs) return;
  const int a = r.seg_adapter[s];
  const int rank = live_rank(L, a, j);
  const int q0 = qc * kGemvRanks;
  if (q0 >= rank) return;
  const int nq = min(kGemvRanks, rank - q0);
  const int rho = rank_offset(L, j);
  const int p_begin = r.seg_start[s], p_end = r.seg_start[s + 1];
  const uint16_t* A = L.pool + (int64_t)a * L.pool_stride + L.off_a + (int64_t)(rho + q0) * k;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int kw = k / 8;
  for (int pc = p_begin; pc < p_end; pc += kGemvRows) {
    const int rows = min(kGemvRows, p_end - pc);
    const uint16_t* xr[kGemvRows];
#pragma unroll
    for (int rr = 0; rr < kGemvRows; ++rr)  // rows past the segment repeat its last row; their sums are dropped
      xr[rr] = x + (int64_t)r.tok_perm[pc + min(rr, rows - 1)] * x_stride;
    float v[kGemvRows * kGemvRanks];
#pragma unroll
    for (int i = 0; i < kGemvRows * kGemvRanks; ++i) v[i] = 0.0f;
    for (int i = tid; i < kw; i += kGemvThreads) {
      uint4 xv[kGemvRows];
#pragma unroll
      for (int rr = 0; rr < kGemvRows; ++rr) xv[rr] = *reinterpret_cast<const uint4*>(xr[rr] + 8 * i);
#pragma unroll
      for (int q = 0; q < kGemvRanks; ++q) {
        if (q < nq) {
          const uint4 av = *reinterpret_cast<const uint4*>(A + (int64_t)q * k + 8 * i);
#pragma unroll
          for (int rr = 0; rr < kGemvRows; ++rr) v[rr * kGemvRanks + q] = dot8(xv[rr], av, v[rr * kGemvRanks + q]);
        }
      }
    }
    // reduce-scatter across the wave: afterwards lane l holds the wave's sum of value l (row l/16, rank l%16)
#pragma unroll
    for (int h = 32; h >= 1; h >>= 1) {
      const bool upper = (lane & h) != 0;
#pragma unroll
      for (int i = 0; i < h; ++i) {
        const float send = upper ? v[i] : v[i + h];
        const float keep = upper ? v[i + h] : v[i];
        v[i] = keep + __shfl_xor(send, h);
      }
    }
    red[wave][lane] = v[0];
    __syncthreads();
    if (wave == 0) {
      const float sum = ((red[0][lane] + red[1][lane]) + red[2][lane]) + red[3][lane];
      const int rr = lane / kGemvRanks, q = lane % kGemvRanks;
      if (rr < rows && q < nq) mid[(int64_t)(pc + rr) * L.rank_cap + rho + q0 + q] = f32_to_bf16(sum);
    }
    __syncthreads();
  }
}

constexpr int kSM = 64;          // sorted positions per workgroup
constexpr int kSK = 64;          // inputs per staged chunk
constexpr int kSLd = kSK + 8;    // LDS row stride in bf16 (144 bytes: 16-byte reads of 32 rows hit distinct banks)
constexpr int kJobsPerWave = 2;  // (row block, matrix, 32-rank block) accumulators per wave and round

__global__ __launch_bounds__(256) void shrink_mfma_kernel(mlora_lora_t L, mlora_route_t r,
                                                         const uint16_t* __restrict__ x, int64_t x_stride, int32_t k,
                                                         uint16_t* __restrict__ mid) {
  __shared__ __attribute__((aligned(16))) uint16_t xs[kSM * kSLd];
  const int64_t T = r.tokens;
  const int64_t p0 = (int64_t)blockIdx.x * kSM;
  if (p0 >= T) return;
  const int nseg = *r.num_segs;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int64_t tile_end = min(p0 + kSM, T);
  const int srow = tid >> 2, scol = (tid & 3) * 16;  // staging: 16 inputs of one row per thread
  const int64_t sp = p0 + srow;
  for (int s = segment_of(r.seg_start, nseg, p0); s < nseg && r.seg_start[s] < tile_end; ++s) {
    const int64_t sb = max((int64_t)r.seg_start[s], p0), se = min((int64_t)r.seg_start[s + 1], tile_end);
    if (se <= sb) continue;
    const int a = r.seg_adapter[s];
    int rank[MLORA_MAX_MATS];
    int blocks_total = 0;
    for (int j = 0; j < L.n_mats; ++j) {
      rank[j] = live_rank(L, a, j);
      blocks_total += (rank[j] + 31) >> 5;
    }
    const int rb_lo = (int)((sb - p0) >> 5), rb_hi = (int)((se - 1 - p0) >> 5);
    const int njobs = (rb_hi - rb_lo + 1) * blocks_total;
    if (njobs == 0) continue;
    const bool stage = sp >= sb && sp < se;
    const uint16_t* xsrc = stage ? x + (int64_t)r.tok_perm[sp] * x_stride + scol : nullptr;
    const uint16_t* Abase = L.pool + (int64_t)a * L.pool_stride + L.off_a;
    for (int round = 0; round < njobs; round += 4 * kJobsPerWave) {
      f32x16_t acc[kJobsPerWave];
      int jrow[kJobsPerWave], jmat[kJobsPerWave], jn[kJobsPerWave];
      bool jok[kJobsPerWave];
      const uint16_t* arow[kJobsPerWave];
#pragma unroll
      for (int jj = 0; jj < kJobsPerWave; ++jj) {
        acc[jj] = f32x16_t{};
        const int job = round + wave + 4 * jj;
        jok[jj] = job < njobs;
        int rbi = 0, j = 0, kb = 0;
        if (jok[jj]) {
          rbi = job / blocks_total;
          int b = job - rbi * blocks_total;
          while (b >= ((rank[j] + 31) >> 5)) {
            b -= (rank[j] + 31) >> 5;
            ++j;
          }
          kb = b;
        }
        jrow[jj] = (rb_lo + rbi) * 32;
        jmat[jj] = j;
        jn[jj] = kb * 32 + (lane & 31);  // this lane's rank (MFMA column)
        const bool nok = jok[jj] && jn[jj] < rank[j];
        arow[jj] = nok ? Abase + (int64_t)(rank_offset(L, j) + jn[jj]) * k : nullptr;
      }
      for (int kc = 0; kc < k; kc += kSK) {
        __syncthreads();
        uint4 v0 = make_uint4(0, 0, 0, 0), v1 = v0;
        if (xsrc != nullptr) {
          v0 = *reinterpret_cast<const uint4*>(xsrc + kc);
          v1 = *reinterpret_cast<const uint4*>(xsrc + kc + 8);
        }
        *reinterpret_cast<uint4*>(&xs[srow * kSLd + scol]) = v0;
        *reinterpret_cast<uint4*>(&xs[srow * kSLd + scol + 8]) = v1;
        __syncthreads();
#pragma unroll
        for (int jj = 0; jj < kJobsPerWave; ++jj) {
          if (!jok[jj]) continue;
#pragma unroll
          for (int k16 = 0; k16 < kSK / 16; ++k16) {
            const int kk = k16 * 16 + (lane >> 5) * 8;
            const uint4 av = *reinterpret_cast<const uint4*>(&xs[(jrow[jj] + (lane & 31)) * kSLd + kk]);
            const uint4 bv = arow[jj] != nullptr ? *reinterpret_cast<const uint4*>(arow[jj] + kc + kk)
                                                  : make_uint4(0, 0, 0, 0);
            acc[jj] = mfma32(av, bv, acc[jj]);
          }
        }
      }
#pragma unroll
      for (int jj = 0; jj < kJobsPerWave; ++jj) {
        if (!jok[jj] || jn[jj] >= rank[jmat[jj]]) continue;
        uint16_t* out = mid + rank_offset(L, jmat[jj]) + jn[jj];
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          const int64_t p = p0 + jrow[jj] + (i >> 2) * 8 + (lane >> 5) * 4 + (i & 3);
          if (p >= sb && p < se) out[p * L.rank_cap] = f32_to_bf16(acc[jj][i]);
        }
      }
    }
  }
}

}  // namespace

int launch_shrink(const mlora_lora_t& L, const mlora_route_t& r, const uint16_t* x, int64_t x_stride, int32_t k,
                    uint16_t* mid, bool mfma, hipStream_t stream) {
  if (r.tokens == 0 || r.max_segs == 0) return MLORA_OK;
  if (mfma) {
    const int64_t blocks = (r.tokens + kSM - 1) / kSM;
    hipLaunchKernelGGL(shrink_mfma_kernel, dim3((unsigned)blocks), dim3(256), 0, stream, L, r, x, x_stride, k, mid);
  } else {
    int maxcap = 0;
    for (int j = 0; j < L.n_mats; ++j) maxcap = L.cap[j] > maxcap ? L.cap[j] : maxcap;
    const int qchunks = (maxcap + kGemvRanks - 1) / kGemvRanks;
    const int64_t blocks = (int64_t)r.max_segs * L.n_mats * qchunks;
    if (blocks == 0) return MLORA_OK;
    hipLaunchKernelGGL(shrink_gemv_kernel, dim3((unsigned)blocks), dim3(kGemvThreads), 0, stream, L, r, x, x_stride,
                       k, mid, qchunks);
  }
  return hipGetLastError() == hipSuccess ? MLORA_OK : MLORA_ELAUNCH;
}
