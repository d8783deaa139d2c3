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
      // every load is issued before any use (rank rows past the live rank re-read the last live row and are dropped),
      // so the 4 + 16 requests of a thread are in flight together
      uint4 xv[kGemvRows], av[kGemvRanks];
#pragma unroll
      for (int rr = 0; rr < kGemvRows; ++rr) xv[rr] = *reinterpret_cast<const uint4*>(xr[rr] + 8 * i);
#pragma unroll
      for (int q = 0; q < kGemvRanks; ++q)
        av[q] = *reinterpret_cast<const uint4*>(A + (int64_t)min(q, nq - 1) * k + 8 * i);
#pragma unroll
      for (int q = 0; q < kGemvRanks; ++q)
#pragma unroll
        for (int rr = 0; rr < kGemvRows; ++rr) v[rr * kGemvRanks + q] = dot8(xv[rr], av[q], v[rr * kGemvRanks + q]);
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

constexpr int kSM = 64;         // sorted positions per workgroup: 2 row blocks of 32
constexpr int kSK = 64;         // inputs per step
constexpr int kSLd = kSK + 8;   // LDS row stride in bf16 (144 bytes: 16-byte reads of 32 rows hit distinct banks)
constexpr int kMaxBlocks = 8;   // 32-rank blocks per pass (256 ranks)

// The (matrix, 32-rank block) of block index b of an adapter whose live ranks are rk[].
__device__ __forceinline__ void rank_block(const int* rk, int n_mats, int b, int& j, int& kb) {
  j = 0;
  while (j + 1 < n_mats && b >= ((rk[j] + 31) >> 5)) {
    b -= (rk[j] + 31) >> 5;
    ++j;
  }
  kb = b;
}

// One workgroup per 64 sorted positions and every segment crossing them: x rows and the segment's A rows are staged
// through double-buffered LDS (the next step's loads in flight while the MFMAs run, one barrier per step); waves
// (row block rb, half) take the rank blocks of their half.
__global__ __launch_bounds__(256) void shrink_mfma_kernel(mlora_lora_t L, mlora_route_t r,
                                                         const uint16_t* __restrict__ x, int64_t x_stride, int32_t k,
                                                         uint16_t* __restrict__ mid) {
  __shared__ __attribute__((aligned(16))) uint16_t xs[2][kSM * kSLd];
  __shared__ __attribute__((aligned(16))) uint16_t as[2][kMaxBlocks * 32 * kSLd];
  const int64_t T = r.tokens;
  const int64_t p0 = (int64_t)blockIdx.x * kSM;
  if (p0 >= T) return;
  const int nseg = *r.num_segs;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int rb = wave & 1, half = wave >> 1;
  const int64_t tile_end = min(p0 + kSM, T);
  const int srow = tid >> 2, scol = (tid & 3) * 16;  // x staging: 16 inputs of one row
  const int arow = tid >> 3, acol = (tid & 7) * 8;   // A staging: 8 inputs of one rank row per block
  const int64_t sp = p0 + srow;
  const int nk = k / kSK;
  for (int s = segment_of(r.seg_start, nseg, p0); s < nseg && r.seg_start[s] < tile_end; ++s) {
    const int64_t sb = max((int64_t)r.seg_start[s], p0), se = min((int64_t)r.seg_start[s + 1], tile_end);
    if (se <= sb) continue;
    const int a = r.seg_adapter[s];
    int rk[MLORA_MAX_MATS];
    int nblk = 0;
    for (int j = 0; j < L.n_mats; ++j) {
      rk[j] = live_rank(L, a, j);
      nblk += (rk[j] + 31) >> 5;
    }
    if (nblk == 0) continue;
    const uint16_t* xsrc = (sp >= sb && sp < se) ? x + (int64_t)r.tok_perm[sp] * x_stride + scol : nullptr;
    const uint16_t* Abase = L.pool + (int64_t)a * L.pool_stride + L.off_a;
    for (int b0 = 0; b0 < nblk; b0 += kMaxBlocks) {
      const int nbp = min(kMaxBlocks, nblk - b0);
      const uint16_t* asrc[kMaxBlocks];
#pragma unroll
      for (int bi = 0; bi < kMaxBlocks; ++bi) {
        asrc[bi] = nullptr;
        if (bi < nbp) {
          int j, kb;
          rank_block(rk, L.n_mats, b0 + bi, j, kb);
          const int n = kb * 32 + arow;
          if (n < rk[j]) asrc[bi] = Abase + (int64_t)(rank_offset(L, j) + n) * k + acol;
        }
      }
      uint4 xv[2], av[kMaxBlocks];
      auto fetch = [&](int kc) {
        xv[0] = xv[1] = make_uint4(0, 0, 0, 0);
        if (xsrc != nullptr) {
          xv[0] = *reinterpret_cast<const uint4*>(xsrc + kc);
          xv[1] = *reinterpret_cast<const uint4*>(xsrc + kc + 8);
        }
#pragma unroll
        for (int bi = 0; bi < kMaxBlocks; ++bi)
          av[bi] = asrc[bi] != nullptr ? *reinterpret_cast<const uint4*>(asrc[bi] + kc) : make_uint4(0, 0, 0, 0);
      };
      auto stage = [&](int buf) {
        *reinterpret_cast<uint4*>(&xs[buf][srow * kSLd + scol]) = xv[0];
        *reinterpret_cast<uint4*>(&xs[buf][srow * kSLd + scol + 8]) = xv[1];
#pragma unroll
        for (int bi = 0; bi < kMaxBlocks; ++bi)
          if (bi < nbp) *reinterpret_cast<uint4*>(&as[buf][(bi * 32 + arow) * kSLd + acol]) = av[bi];
      };
      f32x16_t acc[kMaxBlocks / 2];
#pragma unroll
      for (int m = 0; m < kMaxBlocks / 2; ++m) acc[m] = f32x16_t{};
      fetch(0);
      stage(0);
      if (nk > 1) fetch(kSK);
      __syncthreads();
      for (int it = 0; it < nk; ++it) {
        const int cur = it & 1;
#pragma unroll
        for (int k16 = 0; k16 < kSK / 16; ++k16) {
          const int kk = k16 * 16 + (lane >> 5) * 8;
          const uint4 av16 = *reinterpret_cast<const uint4*>(&xs[cur][(rb * 32 + (lane & 31)) * kSLd + kk]);
#pragma unroll
          for (int m = 0; m < kMaxBlocks / 2; ++m) {
            const int bi = half + 2 * m;
            if (bi < nbp) {
              const uint4 bv = *reinterpret_cast<const uint4*>(&as[cur][(bi * 32 + (lane & 31)) * kSLd + kk]);
              acc[m] = mfma32(av16, bv, acc[m]);
            }
          }
        }
        if (it + 1 < nk) stage(cur ^ 1);
        if (it + 2 < nk) fetch((it + 2) * kSK);
        __syncthreads();
      }
#pragma unroll
      for (int m = 0; m < kMaxBlocks / 2; ++m) {
        const int bi = half + 2 * m;
        if (bi >= nbp) continue;
        int j, kb;
        rank_block(rk, L.n_mats, b0 + bi, j, kb);
        const int n = kb * 32 + (lane & 31);
        if (n >= rk[j]) continue;
        uint16_t* out = mid + rank_offset(L, j) + n;
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          const int64_t p = p0 + rb * 32 + (i >> 2) * 8 + (lane >> 5) * 4 + (i & 3);
          if (p >= sb && p < se) out[p * L.rank_cap] = f32_to_bf16(acc[m][i]);
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
