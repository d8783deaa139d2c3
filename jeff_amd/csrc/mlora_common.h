// Device helpers shared by the gfx950 kernels of the multi-LoRA INT4 linear.
#pragma once

#include <hip/hip_runtime.h>
#include <climits>
#include <stdint.h>

#include "jeff_mlora.h"

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));

namespace mlora {

constexpr int kWave = 64;

__device__ __forceinline__ float bf16_to_f32(uint32_t h) { return __uint_as_float(h << 16); }
__device__ __forceinline__ float bf16_lo(uint32_t v) { return __uint_as_float(v << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t v) { return __uint_as_float(v & 0xFFFF0000u); }

// Two float32 values rounded to nearest even and packed as bf16 (lo in bits 0..15): one v_cvt_pk_bf16_f32.
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  bf16x2_t v = {(__bf16)lo, (__bf16)hi};
  return __builtin_bit_cast(uint32_t, v);
}
__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
  __bf16 b = (__bf16)f;
  return __builtin_bit_cast(uint16_t, b);
}

// The 8 weights of one packed word (input j of the 8 in bits 4j..4j+3) as bf16((c - z) s), in input order.
// fma(c, s, -z s) is exact for every finite scale below 2^120: c s and z s are products of a 4-bit integer and an
// 8-bit significand, and their difference has at most 13 significant bits, so the single rounding to bf16 is the
// only one. zs = z * s is formed once per (group, column) by the caller.
__device__ __forceinline__ uint4 dequant_word(uint32_t w, float s, float zs) {
  uint32_t lo = w & 0x0F0F0F0Fu;         // codes of inputs 0, 2, 4, 6 in bytes 0..3
  uint32_t hi = (w >> 4) & 0x0F0F0F0Fu;  // codes of inputs 1, 3, 5, 7
  // keep the byte layout visible to the compiler so each code converts with one v_cvt_f32_ubyteN
  asm volatile("" : "+v"(lo));
  asm volatile("" : "+v"(hi));
  const float c0 = (float)(lo & 0xFF), c2 = (float)((lo >> 8) & 0xFF);
  const float c4 = (float)((lo >> 16) & 0xFF), c6 = (float)(lo >> 24);
  const float c1 = (float)(hi & 0xFF), c3 = (float)((hi >> 8) & 0xFF);
  const float c5 = (float)((hi >> 16) & 0xFF), c7 = (float)(hi >> 24);
  uint4 r;
  r.x = pack_bf16x2(__builtin_fmaf(c0, s, -zs), __builtin_fmaf(c1, s, -zs));
  r.y = pack_bf16x2(__builtin_fmaf(c2, s, -zs), __builtin_fmaf(c3, s, -zs));
  r.z = pack_bf16x2(__builtin_fmaf(c4, s, -zs), __builtin_fmaf(c5, s, -zs));
  r.w = pack_bf16x2(__builtin_fmaf(c6, s, -zs), __builtin_fmaf(c7, s, -zs));
  return r;
}

// Keep the first n of 8 packed bf16 values, zero the rest (n <= 0: all zero, n >= 8: unchanged).
__device__ __forceinline__ uint4 keep_first(uint4 v, int n) {
  if (n >= 8) return v;
  uint32_t e[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int lo = 2 * i, hi = 2 * i + 1;
    uint32_t m = (lo < n ? 0x0000FFFFu : 0u) | (hi < n ? 0xFFFF0000u : 0u);
    e[i] &= m;
  }
  return make_uint4(e[0], e[1], e[2], e[3]);
}

__device__ __forceinline__ bf16x8_t as_bf16x8(uint4 v) { return __builtin_bit_cast(bf16x8_t, v); }

// The gated activation of packed bf16 values (the reference's silu_mul, engine/fast_path.py:141-156): for gate g and
// up u, bf16(bf16(g / (1 + exp(-g))) u), each value independently. Shared by silu_mul_kernel and the products that
// apply it in their output tiles, so both give the same bits. The quotient g / d is the hardware reciprocal's q0 =
// g rcp(d) corrected once by its exact residual (fma(-q0, d, g), exact while q0 is within a few ulps of g / d):
// q0 + residual rcp(d), rounded once, is the correctly rounded quotient except within about 2^-22 ulp of a rounding
// boundary (a bare reciprocal, within 1 ulp, misrounds values within an ulp of a bf16 rounding midpoint). Where d
// reaches 2^120 (g below about -83: the reciprocal would fall among the denormals, which it flushes) the quotient is
// an IEEE division. Where q0 is a zero, an infinity or NaN (g = +-0, +inf, NaN) q0 itself is the quotient: the
// correction step would turn -0 into +0 and +inf into NaN.
__device__ __forceinline__ float bf16_round(float v) {
  return __uint_as_float((uint32_t)__builtin_bit_cast(uint16_t, (__bf16)v) << 16);
}
__device__ __forceinline__ float silu_quotient(float g) {
  const float d = 1.0f + __expf(-g);
  if (__builtin_expect(!(d < 0x1p120f), 0)) return g / d;
  const float r = __builtin_amdgcn_rcpf(d);
  const float q0 = g * r;
  const float q = __builtin_fmaf(__builtin_fmaf(-q0, d, g), r, q0);
  // classes: signalling/quiet NaN (bits 0, 1), -inf (2), -0 (5), +0 (6), +inf (9)
  return __builtin_amdgcn_class(q0, 0x3 | 0x4 | 0x20 | 0x40 | 0x200) ? q0 : q;
}
__device__ __forceinline__ uint4 silu_mul8(uint4 g, uint4 u) {
  const uint32_t gw[4] = {g.x, g.y, g.z, g.w}, uw[4] = {u.x, u.y, u.z, u.w};
  uint32_t o[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const float g0 = bf16_lo(gw[e]), g1 = bf16_hi(gw[e]);
    o[e] = pack_bf16x2(bf16_round(silu_quotient(g0)) * bf16_lo(uw[e]), bf16_round(silu_quotient(g1)) * bf16_hi(uw[e]));
  }
  return make_uint4(o[0], o[1], o[2], o[3]);
}
// four values (two packed pairs each of gate and up)
__device__ __forceinline__ uint2 silu_mul4(uint2 g, uint2 u) {
  const uint4 v = silu_mul8(make_uint4(g.x, g.y, 0, 0), make_uint4(u.x, u.y, 0, 0));
  return make_uint2(v.x, v.y);
}

// The residual add of add_rms (engine/fast_path.py:87-89: x = bf16(x + d)) on packed bf16 pairs: r the residual, v
// the product's output, already rounded once to bf16; the float32 sum rounded to bf16.
__device__ __forceinline__ uint32_t add_bf16x2(uint32_t r, uint32_t v) {
  return pack_bf16x2(bf16_lo(r) + bf16_lo(v), bf16_hi(r) + bf16_hi(v));
}
__device__ __forceinline__ uint16_t add_bf16(uint16_t r, uint16_t v) {
  return (uint16_t)add_bf16x2(r, v);
}

// Output flags the store paths of the product kernels take in one word: bit 0 whole-vector stores are aligned, bit 1
// the residual add (the output rows hold the residual on entry and receive bf16(residual + output)).
constexpr int32_t kStoreVec = 1, kStoreResidual = 2;

// Four consecutive output columns of one row (two packed bf16 pairs lo, hi) to y at yr and, when `last` is not null,
// to the request's last-token row; `left` columns of the row remain from the first. With kStoreResidual the four
// values written are bf16(yr[e] + value), read from the row first.
__device__ __forceinline__ void store4(uint16_t* yr, uint16_t* last, uint32_t lo, uint32_t hi, int left,
                                       int32_t flags) {
  if ((flags & kStoreVec) && left >= 4) {
    if (flags & kStoreResidual) {
      const uint2 rv = *reinterpret_cast<const uint2*>(yr);
      lo = add_bf16x2(rv.x, lo);
      hi = add_bf16x2(rv.y, hi);
    }
    *reinterpret_cast<uint2*>(yr) = make_uint2(lo, hi);
    if (last != nullptr) *reinterpret_cast<uint2*>(last) = make_uint2(lo, hi);
  } else {
    const uint16_t h[4] = {(uint16_t)lo, (uint16_t)(lo >> 16), (uint16_t)hi, (uint16_t)(hi >> 16)};
    for (int e = 0; e < 4 && e < left; ++e) {
      const uint16_t v = (flags & kStoreResidual) ? add_bf16(yr[e], h[e]) : h[e];
      yr[e] = v;
      if (last != nullptr) last[e] = v;
    }
  }
}

__device__ __forceinline__ f32x16_t mfma32(uint4 a, uint4 b, f32x16_t c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(as_bf16x8(a), as_bf16x8(b), c, 0, 0, 0);
}

// 8 products of bf16 pairs accumulated into acc with v_dot2_f32_bf16, in pair order.
__device__ __forceinline__ float dot8(uint4 a, uint4 b, float acc) {
  acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, a.x), __builtin_bit_cast(bf16x2_t, b.x), acc,
                                        false);
  acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, a.y), __builtin_bit_cast(bf16x2_t, b.y), acc,
                                        false);
  acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, a.z), __builtin_bit_cast(bf16x2_t, b.z), acc,
                                        false);
  acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, a.w), __builtin_bit_cast(bf16x2_t, b.w), acc,
                                        false);
  return acc;
}

// The segment s with seg_start[s] <= p < seg_start[s + 1], for 0 <= p < seg_start[nseg] (binary search).
__device__ __forceinline__ int segment_of(const int32_t* seg_start, int nseg, int64_t p) {
  int lo = 0, hi = nseg - 1;
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (seg_start[mid] <= p) lo = mid; else hi = mid - 1;
  }
  return lo;
}

// Live rank of matrix j in pool row a, clamped to [0, cap] so a corrupt table cannot move a read out of the row.
__device__ __forceinline__ int live_rank(const mlora_lora_t& L, int a, int j) {
  int r = L.ranks[(int64_t)a * L.ranks_stride + j];
  r = r < 0 ? 0 : r;
  return r > L.cap[j] ? L.cap[j] : r;
}

// Row stride (elements) of sB_j in a pool row whose live rank of matrix j is `rank`: the rank rounded up to a power
// of two, at least 8, at most cap_j (a rank-0 row keeps stride min(8, cap_j), so reads that ignore the rank stay in
// the block). Low-rank adapters' rows are then dense: a rank-8 row is 16 bytes, not cap_j * 2.
__device__ __forceinline__ int sb_stride(int rank, int cap) {
  const int s = rank <= 8 ? 8 : 1 << (32 - __builtin_clz((unsigned)(rank - 1)));
  return s < cap ? s : cap;
}

// Stacked-rank offset rho_j and output-column offset of matrix j.
__device__ __forceinline__ int rank_offset(const mlora_lora_t& L, int j) {
  int o = 0;
  for (int i = 0; i < j; ++i) o += L.cap[i];
  return o;
}
__device__ __forceinline__ int col_offset(const mlora_lora_t& L, int j) {
  int o = 0;
  for (int i = 0; i < j; ++i) o += L.cols[i];
  return o;
}
// The matrix whose output columns hold column c (c < sum of cols).
__device__ __forceinline__ int matrix_of(const mlora_lora_t& L, int c) {
  int j = 0, o = L.cols[0];
  while (j + 1 < L.n_mats && c >= o) {
    ++j;
    o += L.cols[j];
  }
  return j;
}

}  // namespace mlora

// The decision head: option logits per row from its adapter's readout; the masked, tempered softmax.
int launch_readout_logits(const uint16_t* hidden, int64_t hidden_stride, int32_t dim, const uint16_t* pool,
                          int64_t pool_stride, int32_t options, int32_t pool_rows, const int32_t* adapters,
                          int32_t rows, float* logits, hipStream_t stream);
int launch_option_softmax(const float* logits, int32_t options, const int32_t* adapters, const int32_t* counts,
                          const float* temp_pool, int32_t pool_rows, int32_t rows, float* probs, hipStream_t stream);
// The element-wise work around the linear: residual add + RMSNorm; SiLU of the gate half times the up half.
int launch_add_rms(const uint16_t* x, int64_t x_stride, const uint16_t* d, int64_t d_stride, const float* w1,
                   uint16_t* xo, int64_t xo_stride, uint16_t* h, int64_t h_stride, int64_t rows, int32_t n, float eps,
                   hipStream_t stream);
int launch_silu_mul(const uint16_t* gu, int64_t gu_stride, uint16_t* y, int64_t y_stride, int64_t rows, int32_t inter,
                    hipStream_t stream);
// The split product's second launch stages its rows' first factors in LDS: at most this stacked rank.
#define MLORA_SPLIT_MAX_RANK 512

// Launchers (one per kernel family), defined in their .hip files; each returns MLORA_OK or MLORA_ELAUNCH.
int launch_route(const int32_t* adp, const int32_t* cu, int32_t row_len, const mlora_route_t& r, int32_t pool_rows,
                 hipStream_t stream);
int launch_dequant(const mlora_int4_t& w, uint16_t* out, hipStream_t stream);
int launch_shrink(const mlora_lora_t& L, const mlora_route_t& r, const uint16_t* x, int64_t x_stride, int32_t k,
                  uint16_t* mid, bool mfma, hipStream_t stream);
// 256 x 256 tiles; with part != nullptr the split mode: ksplit input ranges, float32 sums to part, nothing else.
// inter > 0: a gated product (the group is gate and up, inter columns each; y and last_out receive silu(gate) * up,
// inter columns), fused mode only. residual: y holds the residual rows on entry and receives bf16(residual + output)
// (last_out the same sums), fused mode and not gated.
int launch_base256(const mlora_int4_t& w, const mlora_lora_t& L, const mlora_route_t& r, const uint16_t* x,
                   int64_t x_stride, uint16_t* y, int64_t y_stride, uint16_t* last_out, int32_t n_out,
                   const uint16_t* mid, float* part, int32_t ksplit, hipStream_t stream, int32_t inter = 0,
                   bool residual = false);
// The second launch of a split product: partial sums in order + LoRA term, rounded once (inter > 0: gated, as above;
// the register form's capacities only, finish_registers; residual as above, the register form only, not gated).
bool finish_registers(const mlora_lora_t& L);
int launch_finish(const mlora_lora_t& L, const mlora_route_t& r, const float* part, int32_t ksplit, int32_t ld,
                  const uint16_t* mid, uint16_t* y, int64_t y_stride, uint16_t* last_out, int32_t n_out,
                  hipStream_t stream, int32_t inter = 0, bool residual = false);
// Narrow product (every token, at most 256, in one row tile of 64 columns; inter and residual as above). One input
// range: the tiles add the LoRA term themselves. ksplit > 1 ranges: float32 tiles in part (dec_partials_bytes(w,
// ksplit)), then a second launch adds the ranges and the LoRA term. shrink: the product computes the first factors
// into mid (segment form: their own launch before one range, inside the first launch with ranges); else mid holds
// them.
size_t dec_partials_bytes(const mlora_int4_t& w, int32_t ksplit);
int launch_dec(const mlora_int4_t& w, const mlora_lora_t& L, const mlora_route_t& r, const uint16_t* x,
               int64_t x_stride, uint16_t* y, int64_t y_stride, uint16_t* last_out, int32_t n_out, uint16_t* mid,
               bool shrink, float* part, int32_t ksplit, hipStream_t stream, int32_t inter = 0,
               bool residual = false);
int launch_base(const mlora_int4_t* w, const mlora_lora_t& L, const mlora_route_t& r, const uint16_t* x,
                int64_t x_stride, uint16_t* y, int64_t y_stride, uint16_t* last_out, int32_t n_out,
                const uint16_t* mid, bool gemv, hipStream_t stream);
