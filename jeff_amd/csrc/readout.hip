// The decision head after the last projection: each request row's option logits from its own adapter's readout, then
// the masked, tempered softmax (the reference's readout_rows: engine/batched_kernels.py:492-559, with
// DecisionModel.forward's mask and temperature).
//  - readout_logits_kernel: one workgroup per (row, 64 options); each wave takes 16 options, a lane 16-byte chunks of
//    the hidden vector and of each option's readout row (coalesced across the wave), v_dot2_f32_bf16 into a float32
//    partial, then a fixed shuffle tree across the wave; the sum is rounded to bf16 and stored as float32.
//  - option_softmax_kernel: one wave per row; options from the row's count on get the logit -1e9, the logits are
//    divided by the adapter's temperature and the softmax taken over all options (max and sum by fixed shuffle trees).
#include "mlora_common.h"

namespace {

using namespace mlora;

constexpr int kRoOptionsPerBlock = 64;
constexpr int kRoOptionsPerWave = 16;
constexpr int kRoThreads = 256;
constexpr int kRoGroup = 4;        // options whose readout loads are in flight together
constexpr int kRoMaxChunks = 4;    // 16-byte chunks of the hidden vector per lane: dim <= 64 * 8 * 4 = 2048

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o);
  return v;
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v = fmaxf(v, __shfl_xor(v, o));
  return v;
}

__global__ __launch_bounds__(kRoThreads) void readout_logits_kernel(const uint16_t* __restrict__ hidden,
                                                                   int64_t hidden_stride, int32_t dim,
                                                                   const uint16_t* __restrict__ pool,
                                                                   int64_t pool_stride, int32_t options,
                                                                   int32_t pool_rows,
                                                                   const int32_t* __restrict__ adapters,
                                                                   float* __restrict__ logits) {
  const int b = blockIdx.x;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  int a = adapters[b];
  if (a < 0 || a >= pool_rows) a = 0;  // an index outside the pool reads row 0: every read stays inside the pool
  const uint16_t* h = hidden + (int64_t)b * hidden_stride;
  const uint16_t* w = pool + (int64_t)a * pool_stride;
  const int chunks = dim / 8;  // 16-byte chunks of a row; lane l takes chunks l, l + 64, ...
  uint4 hv[kRoMaxChunks];
#pragma unroll
  for (int j = 0; j < kRoMaxChunks; ++j) {
    const int c = lane + 64 * j;
    hv[j] = c < chunks ? *reinterpret_cast<const uint4*>(h + 8 * c) : make_uint4(0, 0, 0, 0);
  }
  const int o0 = blockIdx.y * kRoOptionsPerBlock + wave * kRoOptionsPerWave;
  for (int g = 0; g < kRoOptionsPerWave; g += kRoGroup) {
    uint4 wv[kRoGroup][kRoMaxChunks];
#pragma unroll
    for (int i = 0; i < kRoGroup; ++i) {
      const int o = min(o0 + g + i, options - 1);  // options past the last re-read it; their sums are not stored
#pragma unroll
      for (int j = 0; j < kRoMaxChunks; ++j) {
        const int c = lane + 64 * j;
        wv[i][j] = c < chunks ? *reinterpret_cast<const uint4*>(w + (int64_t)o * dim + 8 * c) : make_uint4(0, 0, 0, 0);
      }
    }
#pragma unroll
    for (int i = 0; i < kRoGroup; ++i) {
      float acc = 0.0f;
#pragma unroll
      for (int j = 0; j < kRoMaxChunks; ++j) acc = dot8(wv[i][j], hv[j], acc);
      acc = wave_sum(acc);
      const int o = o0 + g + i;
      if (lane == 0 && o < options) logits[(int64_t)b * options + o] = bf16_to_f32(f32_to_bf16(acc));
    }
  }
}

__global__ __launch_bounds__(64) void option_softmax_kernel(const float* __restrict__ logits, int32_t options,
                                                           const int32_t* __restrict__ adapters,
                                                           const int32_t* __restrict__ counts,
                                                           const float* __restrict__ temp_pool, int32_t pool_rows,
                                                           float* __restrict__ out) {
  const int b = blockIdx.x, lane = threadIdx.x;
  int a = adapters[b];
  if (a < 0 || a >= pool_rows) a = 0;
  const int count = counts[b];
  const float t = temp_pool[a];
  constexpr int kPer = 4;  // options per lane: at most 256
  float x[kPer];
  float m = -INFINITY;
#pragma unroll
  for (int k = 0; k < kPer; ++k) {
    const int o = lane + 64 * k;
    float v = -INFINITY;
    if (o < options) {
      v = o < count ? logits[(int64_t)b * options + o] : -1e9f;
      v = v / t;
    }
    x[k] = v;
    m = fmaxf(m, v);
  }
  m = wave_max(m);
  float s = 0.0f;
#pragma unroll
  for (int k = 0; k < kPer; ++k) {
    x[k] = lane + 64 * k < options ? expf(x[k] - m) : 0.0f;
    s += x[k];
  }
  s = wave_sum(s);
#pragma unroll
  for (int k = 0; k < kPer; ++k) {
    const int o = lane + 64 * k;
    if (o < options) out[(int64_t)b * options + o] = x[k] / s;
  }
}

}  // namespace

int launch_readout_logits(const uint16_t* hidden, int64_t hidden_stride, int32_t dim, const uint16_t* pool,
                          int64_t pool_stride, int32_t options, int32_t pool_rows, const int32_t* adapters,
                          int32_t rows, float* logits, hipStream_t stream) {
  if (rows == 0) return MLORA_OK;
  const dim3 grid((unsigned)rows, (unsigned)((options + kRoOptionsPerBlock - 1) / kRoOptionsPerBlock));
  hipLaunchKernelGGL(readout_logits_kernel, grid, dim3(kRoThreads), 0, stream, hidden, hidden_stride, dim, pool,
                     pool_stride, options, pool_rows, adapters, logits);
  return hipGetLastError() == hipSuccess ? MLORA_OK : MLORA_ELAUNCH;
}

int launch_option_softmax(const float* logits, int32_t options, const int32_t* adapters, const int32_t* counts,
                          const float* temp_pool, int32_t pool_rows, int32_t rows, float* probs, hipStream_t stream) {
  if (rows == 0) return MLORA_OK;
  hipLaunchKernelGGL(option_softmax_kernel, dim3((unsigned)rows), dim3(64), 0, stream, logits, options, adapters,
                     counts, temp_pool, pool_rows, probs);
  return hipGetLastError() == hipSuccess ? MLORA_OK : MLORA_ELAUNCH;
}
