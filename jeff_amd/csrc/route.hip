// Adapter routing: request rows -> segments of the sorted order, one segment per adapter present.
// Replaces the reference's per-tile lookup adp[t // row_len] (engine/fast_path.py:167,189;
// engine/int4_kernels.py:72,113) with a stable sort, so every adapter's tokens are contiguous.
#include "mlora_common.h"

namespace {

constexpr int kRouteThreads = 1024;
constexpr int kIndexBits = 13;  // request index in the low bits of a sort key: MLORA_MAX_REQUESTS = 2^13
static_assert((1 << kIndexBits) == MLORA_MAX_REQUESTS, "key layout");
static_assert(MLORA_MAX_POOL_ROWS <= (1 << (31 - kIndexBits)), "a key must stay below the padding key");

// Exclusive prefix sum of one value per thread over the 1024-thread block (16 waves), in thread order.
__device__ int block_exclusive_scan(int v, int* wave_sums, int* total) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  int x = v;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const int y = __shfl_up(x, o);
    if (lane >= o) x += y;
  }
  if (lane == 63) wave_sums[wave] = x;
  __syncthreads();
  if (wave == 0) {
    int w = lane < 16 ? wave_sums[lane] : 0;
#pragma unroll
    for (int o = 1; o < 16; o <<= 1) {
      const int y = __shfl_up(w, o);
      if (lane >= o) w += y;
    }
    if (lane < 16) wave_sums[lane] = w;
  }
  __syncthreads();
  const int before = wave == 0 ? 0 : wave_sums[wave - 1];
  *total = wave_sums[15];
  __syncthreads();
  return before + x - v;
}

__global__ __launch_bounds__(kRouteThreads) void route_kernel(const int32_t* __restrict__ adp,
                                                             const int32_t* __restrict__ cu, int32_t row_len,
                                                             mlora_route_t r, int32_t pool_rows) {
  __shared__ uint32_t keys[MLORA_MAX_REQUESTS];
  __shared__ int32_t pstart[MLORA_MAX_REQUESTS];
  __shared__ int32_t segidx[MLORA_MAX_REQUESTS];  // segment of each sorted request
  __shared__ int32_t wave_sums[16];
  __shared__ int32_t status, seq_ok;
  const int tid = threadIdx.x;
  const int B = r.requests;
  const int64_t T = r.tokens;
  if (tid == 0) {
    status = 0;
    seq_ok = 1;
  }
  __syncthreads();
  if (cu != nullptr) {  // the offsets must start at 0, never decrease and end at the token count
    bool bad = tid == 0 && (cu[0] != 0 || (int64_t)cu[B] != T);
    for (int i = tid; i < B; i += kRouteThreads) bad |= cu[i + 1] < cu[i];
    if (bad) atomicAnd(&seq_ok, 0);
  }
  __syncthreads();
  if (!seq_ok) {  // unusable offsets: identity routing through row 0 (no LoRA), flagged
    for (int64_t p = tid; p < T; p += kRouteThreads) {
      r.tok_perm[p] = (int32_t)p;
      r.last_of[p] = -1;
      r.seg_of[p] = 0;
    }
    for (int i = tid; i < B; i += kRouteThreads) r.req_order[i] = i;
    if (tid == 0) {
      *r.num_segs = 1;
      r.seg_start[0] = 0;
      r.seg_start[1] = (int32_t)T;
      r.seg_adapter[0] = 0;
      *r.status = MLORA_ROUTE_BAD_SEQLENS;
    }
    return;
  }
  int n = 1;
  while (n < B) n <<= 1;
  bool bad_adapter = false;
  for (int i = tid; i < n; i += kRouteThreads) {
    uint32_t key = 0xFFFFFFFFu;  // padding sorts last
    if (i < B) {
      int a = adp[i];
      if (a < 0 || a >= pool_rows) {
        a = 0;
        bad_adapter = true;
      }
      key = ((uint32_t)a << kIndexBits) | (uint32_t)i;  // unique keys: any sort of them is stable
    }
    keys[i] = key;
  }
  if (bad_adapter) atomicOr(&status, MLORA_ROUTE_BAD_ADAPTER);
  __syncthreads();
  for (int k = 2; k <= n; k <<= 1) {  // bitonic sort, ascending
    for (int j = k >> 1; j > 0; j >>= 1) {
      for (int i = tid; i < n; i += kRouteThreads) {
        const int ixj = i ^ j;
        if (ixj > i) {
          const uint32_t a = keys[i], b = keys[ixj];
          const bool up = (i & k) == 0;
          if ((a > b) == up) {
            keys[i] = b;
            keys[ixj] = a;
          }
        }
      }
      __syncthreads();
    }
  }
  // lengths and segment starts of 8 consecutive sorted rows per thread
  constexpr int kPer = MLORA_MAX_REQUESTS / kRouteThreads;
  int len[kPer], ada[kPer], rho[kPer];
  bool first[kPer];
  int lsum = 0, fsum = 0;
#pragma unroll
  for (int e = 0; e < kPer; ++e) {
    const int i = tid * kPer + e;
    len[e] = 0;
    first[e] = false;
    ada[e] = 0;
    rho[e] = 0;
    if (i < B) {
      const uint32_t key = keys[i];
      rho[e] = (int)(key & ((1u << kIndexBits) - 1));
      ada[e] = (int)(key >> kIndexBits);
      len[e] = cu != nullptr ? cu[rho[e] + 1] - cu[rho[e]] : row_len;
      first[e] = i == 0 || (keys[i - 1] >> kIndexBits) != (uint32_t)ada[e];
    }
    lsum += len[e];
    fsum += first[e] ? 1 : 0;
  }
  int ltot, ftot;
  int run = block_exclusive_scan(lsum, wave_sums, &ltot);
  int seg = block_exclusive_scan(fsum, wave_sums, &ftot);
#pragma unroll
  for (int e = 0; e < kPer; ++e) {
    const int i = tid * kPer + e;
    if (i < B) {
      pstart[i] = run;
      r.req_order[i] = rho[e];
      segidx[i] = first[e] ? seg : seg - 1;
      if (first[e]) {
        r.seg_adapter[seg] = ada[e];
        r.seg_start[seg] = run;
        ++seg;
      }
      run += len[e];
    }
  }
  if (tid == 0) {
    *r.num_segs = ftot;
    r.seg_start[ftot] = ltot;
  }
  __syncthreads();
  const int lane = tid & 63, wave = tid >> 6;
  for (int i = wave; i < B; i += kRouteThreads / 64) {  // one request per wave, its tokens across the lanes
    const int q = (int)(keys[i] & ((1u << kIndexBits) - 1));
    const int start = cu != nullptr ? cu[q] : q * row_len;
    const int l = cu != nullptr ? cu[q + 1] - cu[q] : row_len;
    const int ps = pstart[i], sg = segidx[i];
    for (int t = lane; t < l; t += 64) {
      r.tok_perm[ps + t] = start + t;
      r.last_of[ps + t] = t == l - 1 ? q : -1;
      r.seg_of[ps + t] = sg;
    }
  }
  if (tid == 0) *r.status = status;
}

// Passes of at most 64 request rows: one workgroup per request. Wave 0 of every workgroup routes all of them in
// registers (one request per lane, a bitonic sort of the same keys by lane shuffles, prefix sums by shuffles; a few
// hundred instructions, cheaper than sharing the result between workgroups); workgroup 0 writes the per-request and
// per-segment outputs, and after one barrier workgroup b writes the tokens of the request at sorted position b, so
// the token stores spread over as many CUs as there are requests. The outputs are the block kernel's, bit for bit.
constexpr int kSmallRequests = 64;
constexpr int kSmallThreads = 256;

__global__ __launch_bounds__(kSmallThreads) void route_small_kernel(const int32_t* __restrict__ adp,
                                                                   const int32_t* __restrict__ cu, int32_t row_len,
                                                                   mlora_route_t r, int32_t pool_rows) {
  __shared__ int32_t s_start[kSmallRequests], s_len[kSmallRequests], s_ps[kSmallRequests];
  __shared__ int32_t s_seg[kSmallRequests], s_q[kSmallRequests];
  __shared__ int32_t s_ok;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int B = r.requests;
  const int64_t T = r.tokens;
  if (wave == 0) {
    const bool live = lane < B;
    int c0 = 0, c1 = 0;
    bool bad = false;
    if (cu != nullptr) {
      if (live) {
        c0 = cu[lane];
        c1 = cu[lane + 1];
        bad = c1 < c0;
      }
      if (lane == 0) bad = bad || cu[0] != 0 || (int64_t)cu[B] != T;
    }
    const bool seq_ok = __ballot(bad) == 0;
    int a = live ? adp[lane] : 0;
    const bool bad_a = live && (a < 0 || a >= pool_rows);
    if (bad_a) a = 0;
    const int len = cu != nullptr ? c1 - c0 : row_len;
    const int start = cu != nullptr ? c0 : lane * row_len;
    uint32_t key = live ? (((uint32_t)a << kIndexBits) | (uint32_t)lane) : 0xFFFFFFFFu;  // padding sorts last
#pragma unroll
    for (int k = 2; k <= 64; k <<= 1)
#pragma unroll
      for (int j = k >> 1; j > 0; j >>= 1) {
        const uint32_t other = __shfl_xor(key, j);
        const bool up = (lane & k) == 0, lower = (lane & j) == 0;
        key = (lower == up) ? min(key, other) : max(key, other);
      }
    const int q = (int)(key & ((1u << kIndexBits) - 1));  // the request at sorted position `lane`
    const int ada = (int)(key >> kIndexBits);
    const int qlen_any = __shfl(len, q & 63);  // every lane takes part in the shuffle
    const int qlen = live ? qlen_any : 0;
    const int qstart = __shfl(start, q & 63);
    const int prev = __shfl_up(ada, 1);
    const bool first = live && (lane == 0 || prev != ada);
    int lsum = qlen, fsum = first ? 1 : 0;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      const int yl = __shfl_up(lsum, o), yf = __shfl_up(fsum, o);
      if (lane >= o) {
        lsum += yl;
        fsum += yf;
      }
    }
    const int pstart = lsum - qlen, seg = fsum - 1;
    const int nseg = __shfl(fsum, 63), total = __shfl(lsum, 63);
    const bool any_bad_adapter = __ballot(bad_a) != 0;  // every lane takes part in the vote
    const bool lead = blockIdx.x == 0;  // the one workgroup that writes the per-request and per-segment outputs
    if (seq_ok) {
      if (live) {
        if (lead) {
          r.req_order[lane] = q;
          if (first) {
            r.seg_adapter[seg] = ada;
            r.seg_start[seg] = pstart;
          }
        }
        s_start[lane] = qstart;
        s_len[lane] = qlen;
        s_ps[lane] = pstart;
        s_seg[lane] = seg;
        s_q[lane] = q;
      }
      if (lane == 0 && lead) {
        *r.num_segs = nseg;
        r.seg_start[nseg] = total;
        *r.status = any_bad_adapter ? MLORA_ROUTE_BAD_ADAPTER : 0;
      }
    }
    if (lane == 0) s_ok = seq_ok ? 1 : 0;
  }
  __syncthreads();
  if (!s_ok) {  // unusable offsets: identity routing through row 0 (no LoRA), flagged
    for (int64_t p = (int64_t)blockIdx.x * kSmallThreads + tid; p < T; p += (int64_t)gridDim.x * kSmallThreads) {
      r.tok_perm[p] = (int32_t)p;
      r.last_of[p] = -1;
      r.seg_of[p] = 0;
    }
    if (blockIdx.x != 0) return;
    for (int i = tid; i < B; i += kSmallThreads) r.req_order[i] = i;
    if (tid == 0) {
      *r.num_segs = 1;
      r.seg_start[0] = 0;
      r.seg_start[1] = (int32_t)T;
      r.seg_adapter[0] = 0;
      *r.status = MLORA_ROUTE_BAD_SEQLENS;
    }
    return;
  }
  for (int i = blockIdx.x; i < B; i += gridDim.x) {  // one request per workgroup, its tokens across the threads
    const int start = s_start[i], l = s_len[i], ps = s_ps[i], sg = s_seg[i], q = s_q[i];
    for (int t = tid; t < l; t += kSmallThreads) {
      r.tok_perm[ps + t] = start + t;
      r.last_of[ps + t] = t == l - 1 ? q : -1;
      r.seg_of[ps + t] = sg;
    }
  }
}

__global__ __launch_bounds__(256) void dequant_kernel(mlora_int4_t w, uint16_t* __restrict__ out) {
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int words_per_col = w.k / 8;
  if (idx >= (int64_t)words_per_col * w.out) return;
  const int c = (int)(idx / words_per_col), i = (int)(idx % words_per_col);
  const int g = (8 * i) / w.group;
  const float s = mlora::bf16_to_f32(w.scales[(int64_t)g * w.columns + c]);
  const float z = w.zeros != nullptr ? (float)w.zeros[(int64_t)g * w.columns + c] : 8.0f;
  const uint32_t word = (uint32_t)w.words[(int64_t)i * w.columns + c];
  *reinterpret_cast<uint4*>(out + (int64_t)c * w.k + 8 * i) = mlora::dequant_word(word, s, z * s);
}

}  // namespace

int launch_route(const int32_t* adp, const int32_t* cu, int32_t row_len, const mlora_route_t& r, int32_t pool_rows,
                 hipStream_t stream) {
  if (r.requests <= kSmallRequests)
    hipLaunchKernelGGL(route_small_kernel, dim3((unsigned)(r.requests > 1 ? r.requests : 1)), dim3(kSmallThreads), 0, stream, adp,
                       cu, row_len, r, pool_rows);
  else
    hipLaunchKernelGGL(route_kernel, dim3(1), dim3(kRouteThreads), 0, stream, adp, cu, row_len, r, pool_rows);
  return hipGetLastError() == hipSuccess ? MLORA_OK : MLORA_ELAUNCH;
}

int launch_dequant(const mlora_int4_t& w, uint16_t* out, hipStream_t stream) {
  const int64_t n = (int64_t)(w.k / 8) * w.out;
  if (n == 0) return MLORA_OK;
  hipLaunchKernelGGL(dequant_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, stream, w, out);
  return hipGetLastError() == hipSuccess ? MLORA_OK : MLORA_ELAUNCH;
}
