// The element-wise work around the fused linear (the reference's engine/fast_path.py:80-100,141-156):
//  - add_rms_kernel: x' = bf16(x + d) (stored when d is given), h = bf16(x' rsqrt(mean(x'^2) + eps) w1). One wave
//    per row, four rows per workgroup; a lane takes 16-byte chunks l, l + 64, ... of the row, sums its squares in
//    chunk and element order, and the wave adds the lanes' sums by a fixed shuffle tree, so every row's result is the
//    same on every call. The row stays in registers between the two passes (at most MLORA_EPILOGUE_MAX_N inputs).
//  - silu_mul_kernel: y = bf16(bf16(g / (1 + exp(-g))) u) for the gate half g and the up half u of each row of the
//    gate_up product, eight columns per thread.
#include "mlora_common.h"

namespace {

using namespace mlora;

constexpr int kRmsRows = 4;                          // rows (waves) per workgroup
constexpr int kRmsChunks = MLORA_EPILOGUE_MAX_N / 512;  // 16-byte chunks per lane at the largest row
constexpr int kRmsGroup = 2;                            // chunks per lane whose loads are issued together
static_assert(kRmsChunks % kRmsGroup == 0, "whole groups of chunks");

__device__ __forceinline__ float wave_sum_fixed(float v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o);
  return v;
}

__global__ __launch_bounds__(kRmsRows * 64) void add_rms_kernel(const uint16_t* __restrict__ x, int64_t x_stride,
                                                                const uint16_t* __restrict__ d, int64_t d_stride,
                                                                const float* __restrict__ w1,
                                                                uint16_t* __restrict__ xo, int64_t xo_stride,
                                                                uint16_t* __restrict__ h, int64_t h_stride,
                                                                int64_t rows, int32_t n, float eps) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * kRmsRows + (threadIdx.x >> 6);
  if (row >= rows) return;
  const int chunks = n / 8;
  const uint16_t* xr = x + row * x_stride;
  float v[kRmsChunks][8];
  float ss = 0.0f;
  // The lane's chunks are taken kRmsGroup at a time: the group's x and d loads are all issued before the first is
  // used (one memory latency per group, not two per chunk); the sums run in chunk order as before.
#pragma unroll
  for (int i0 = 0; i0 < kRmsChunks; i0 += kRmsGroup) {
    if (lane + 64 * i0 >= chunks) break;
    uint4 xv[kRmsGroup], dv[kRmsGroup];
#pragma unroll
    for (int u = 0; u < kRmsGroup; ++u) {
      const int c = lane + 64 * (i0 + u);
      if (c < chunks) {
        xv[u] = *reinterpret_cast<const uint4*>(xr + 8 * c);
        if (d != nullptr) dv[u] = *reinterpret_cast<const uint4*>(d + row * d_stride + 8 * c);
      }
    }
#pragma unroll
    for (int u = 0; u < kRmsGroup; ++u) {
      const int i = i0 + u, c = lane + 64 * i;
      if (c >= chunks) break;
      const uint32_t xw[4] = {xv[u].x, xv[u].y, xv[u].z, xv[u].w};
#pragma unroll
      for (int e = 0; e < 8; ++e) v[i][e] = (e & 1) ? bf16_hi(xw[e >> 1]) : bf16_lo(xw[e >> 1]);
      if (d != nullptr) {
        const uint32_t dw[4] = {dv[u].x, dv[u].y, dv[u].z, dv[u].w};
        uint32_t ow[4];
#pragma unroll
        for (int e = 0; e < 8; e += 2) {
          const uint32_t p = pack_bf16x2(v[i][e] + bf16_lo(dw[e >> 1]), v[i][e + 1] + bf16_hi(dw[e >> 1]));
          ow[e >> 1] = p;
          v[i][e] = bf16_lo(p);
          v[i][e + 1] = bf16_hi(p);
        }
        *reinterpret_cast<uint4*>(xo + row * xo_stride + 8 * c) = make_uint4(ow[0], ow[1], ow[2], ow[3]);
      }
#pragma unroll
      for (int e = 0; e < 8; ++e) ss = __builtin_fmaf(v[i][e], v[i][e], ss);
    }
  }
  ss = wave_sum_fixed(ss);
  const float r = 1.0f / __builtin_sqrtf(ss / (float)n + eps);
#pragma unroll
  for (int i0 = 0; i0 < kRmsChunks; i0 += kRmsGroup) {
    if (lane + 64 * i0 >= chunks) break;
    float4 wa[kRmsGroup], wb[kRmsGroup];
#pragma unroll
    for (int u = 0; u < kRmsGroup; ++u) {
      const int c = lane + 64 * (i0 + u);
      if (c < chunks) {
        wa[u] = *reinterpret_cast<const float4*>(w1 + 8 * c);
        wb[u] = *reinterpret_cast<const float4*>(w1 + 8 * c + 4);
      }
    }
#pragma unroll
    for (int u = 0; u < kRmsGroup; ++u) {
      const int i = i0 + u, c = lane + 64 * i;
      if (c >= chunks) break;
      const float wv[8] = {wa[u].x, wa[u].y, wa[u].z, wa[u].w, wb[u].x, wb[u].y, wb[u].z, wb[u].w};
      uint32_t hw[4];
#pragma unroll
      for (int e = 0; e < 8; e += 2) hw[e >> 1] = pack_bf16x2(v[i][e] * r * wv[e], v[i][e + 1] * r * wv[e + 1]);
      *reinterpret_cast<uint4*>(h + row * h_stride + 8 * c) = make_uint4(hw[0], hw[1], hw[2], hw[3]);
    }
  }
}

__global__ __launch_bounds__(256) void silu_mul_kernel(const uint16_t* __restrict__ gu, int64_t gu_stride,
                                                       uint16_t* __restrict__ y, int64_t y_stride, int64_t rows,
                                                       int32_t inter) {
  const int chunks = inter / 8;
  const int64_t f = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int64_t row = f / chunks;
  if (row >= rows) return;
  const int c = (int)(f - row * chunks);
  const uint16_t* gr = gu + row * gu_stride;
  const uint4 gv = *reinterpret_cast<const uint4*>(gr + 8 * c);
  const uint4 uv = *reinterpret_cast<const uint4*>(gr + inter + 8 * c);
  *reinterpret_cast<uint4*>(y + row * y_stride + 8 * c) = silu_mul8(gv, uv);
}

}  // namespace

int launch_add_rms(const uint16_t* x, int64_t x_stride, const uint16_t* d, int64_t d_stride, const float* w1,
                   uint16_t* xo, int64_t xo_stride, uint16_t* h, int64_t h_stride, int64_t rows, int32_t n, float eps,
                   hipStream_t stream) {
  if (rows == 0) return MLORA_OK;
  const int64_t blocks = (rows + kRmsRows - 1) / kRmsRows;
  hipLaunchKernelGGL(add_rms_kernel, dim3((unsigned)blocks), dim3(kRmsRows * 64), 0, stream, x, x_stride, d, d_stride,
                     w1, xo, xo_stride, h, h_stride, rows, n, eps);
  return hipGetLastError() == hipSuccess ? MLORA_OK : MLORA_ELAUNCH;
}

int launch_silu_mul(const uint16_t* gu, int64_t gu_stride, uint16_t* y, int64_t y_stride, int64_t rows, int32_t inter,
                    hipStream_t stream) {
  if (rows == 0) return MLORA_OK;
  const int64_t threads = rows * (inter / 8);
  hipLaunchKernelGGL(silu_mul_kernel, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, stream, gu, gu_stride, y,
                     y_stride, rows, inter);
  return hipGetLastError() == hipSuccess ? MLORA_OK : MLORA_ELAUNCH;
}
