// The INT4 base product with the LoRA second factor ("expand") fused into its epilogue:
//   y[perm[p], c] = bf16( sum_k x[perm[p], k] W[c, k]  +  sum_q mid[p, rho_j + q] sB_j[a][c - o_j, q] )
// W[c, k] = bf16((code - z) s) is dequantised in registers from the packed words; the base and the LoRA term are
// accumulated in float32 and rounded once (the reference's cut product, engine/int4_kernels.py:105-129, without its
// float32 partial buffer). Without the base (kBase = false) the kernels compute lora_add: y += the LoRA term, in place
// (engine/fast_path.py:180-203,277-289).
//  - base_mfma: tiles of 128 sorted tokens x 128 columns, 4 waves of 64 x 64, 32x32x16 bf16 MFMA. Each K step of 64
//    stages x (gathered through the sorted order) and the dequantised weights through LDS; the next step's words and
//    activations are fetched into registers while the MFMAs run.
//  - base_gemv: at most 8 tokens (decode of a few rows). 64 input slices x 16 columns per workgroup, x staged in LDS
//    by chunks of 2048 inputs, each weight word dequantised once and dotted with every token (v_dot2_f32_bf16),
//    slices summed in a fixed order in LDS.
#include "tile_common.h"

namespace {

using namespace mlora;

constexpr int kBM = 128, kBN = 128, kBK = 64;
constexpr int kLd = kBK + 8;  // LDS row stride in bf16: 144 bytes, so 16-byte reads of 32 rows hit distinct banks

// Adds each token's LoRA second product into a wave's accumulators. acc[mb][nb] holds sorted rows
// prow + 32 mb .. +31 and columns pcol + 32 nb .. +31 in the 32x32 MFMA layout. The A operand is the token's first
// factor (mid, zero for rows outside the segment and ranks past the live rank), the B operand the column's rank
// vector of sB_j (zero for columns of other matrices), so one MFMA per 16 ranks adds exact zeros elsewhere.
__device__ __forceinline__ void expand_into(f32x16_t (&acc)[2][2], int64_t prow, int pcol, const mlora_lora_t& L,
                                            const mlora_route_t& r, const uint16_t* __restrict__ mid, int n_out,
                                            int lane) {
  const int64_t T = r.tokens;
  const int nseg = *r.num_segs;
#pragma unroll
  for (int mb = 0; mb < 2; ++mb) {
    const int64_t r0 = prow + mb * 32;
    if (r0 >= T) break;
    const int64_t r1 = min(r0 + 32, T);
    const int64_t row = r0 + (lane & 31);
    for (int s = segment_of(r.seg_start, nseg, r0); s < nseg && r.seg_start[s] < r1; ++s) {
      const int a = r.seg_adapter[s];
      if (a == 0) continue;  // pool row 0 is the base: no update
      const bool rowok = row >= r.seg_start[s] && row < r.seg_start[s + 1];
      const uint16_t* prow_pool = L.pool + (int64_t)a * L.pool_stride;
#pragma unroll
      for (int nb = 0; nb < 2; ++nb) {
        const int c0 = pcol + nb * 32;
        if (c0 >= n_out) break;
        const int c = c0 + (lane & 31);
        const int jlo = matrix_of(L, c0), jhi = matrix_of(L, min(c0 + 31, n_out - 1));
        for (int j = jlo; j <= jhi; ++j) {
          const int rank = live_rank(L, a, j);
          if (rank == 0) continue;
          const int oj = col_offset(L, j);
          const bool colok = c >= oj && c < oj + L.cols[j] && c < n_out;
          const uint16_t* brow = prow_pool + L.off_b[j] + (int64_t)(colok ? c - oj : 0) * sb_stride(rank, L.cap[j]);
          const uint16_t* mrow = mid + (rowok ? row : 0) * L.rank_cap + rank_offset(L, j);
          for (int k0 = 0; k0 < rank; k0 += 16) {
            const int kk = k0 + (lane >> 5) * 8;
            const int nvalid = rank - kk;
            uint4 av = make_uint4(0, 0, 0, 0), bv = av;
            if (nvalid > 0) {
              if (rowok) av = keep_first(*reinterpret_cast<const uint4*>(mrow + kk), nvalid);
              if (colok) bv = keep_first(*reinterpret_cast<const uint4*>(brow + kk), nvalid);
            }
            acc[mb][nb] = mfma32(av, bv, acc[mb][nb]);
          }
        }
      }
    }
  }
}

template <bool kBase>
__global__ __launch_bounds__(256) void base_mfma_kernel(mlora_int4_t w, mlora_lora_t L, mlora_route_t r,
                                                       const uint16_t* __restrict__ x, int64_t x_stride,
                                                       uint16_t* __restrict__ y, int64_t y_stride,
                                                       uint16_t* __restrict__ last_out, int32_t n_out,
                                                       const uint16_t* __restrict__ mid, int32_t m_tiles) {
  __shared__ __attribute__((aligned(16))) uint16_t xs[kBM * kLd];
  __shared__ __attribute__((aligned(16))) uint16_t wsm[kBN * kLd];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int mt = blockIdx.x % m_tiles, nt = blockIdx.x / m_tiles;  // neighbours share a column tile (its weights)
  const int64_t p0 = (int64_t)mt * kBM;
  const int n0 = nt * kBN;
  const int64_t T = r.tokens;
  f32x16_t acc[2][2];
#pragma unroll
  for (int mb = 0; mb < 2; ++mb)
#pragma unroll
    for (int nb = 0; nb < 2; ++nb) acc[mb][nb] = f32x16_t{};

  if constexpr (kBase) {
    const int xr = tid >> 1, xh = (tid & 1) * 32;  // x staging: 32 inputs of one row per thread
    const int64_t xp = p0 + xr;
    const uint16_t* xsrc = xp < T ? x + (int64_t)r.tok_perm[xp] * x_stride + xh : nullptr;
    const int wc = tid & (kBN - 1), wr0 = (tid >> 7) * 4;  // weight staging: 4 words (32 inputs) of one column
    const int col = n0 + wc;
    const bool colok = col < w.columns;
    uint4 xreg[4];
    uint32_t wreg[4];
    float sc = 1.0f, zsc = 8.0f;
    auto fetch = [&](int kc) {
#pragma unroll
      for (int i = 0; i < 4; ++i)
        xreg[i] = xsrc != nullptr ? *reinterpret_cast<const uint4*>(xsrc + kc + 8 * i) : make_uint4(0, 0, 0, 0);
      if (colok) {
#pragma unroll
        for (int i = 0; i < 4; ++i) wreg[i] = (uint32_t)w.words[(int64_t)(kc / 8 + wr0 + i) * w.columns + col];
        const int64_t g = (int64_t)(kc / w.group) * w.columns + col;
        sc = bf16_to_f32(w.scales[g]);
        zsc = (w.zeros != nullptr ? (float)w.zeros[g] : 8.0f) * sc;
      } else {
#pragma unroll
        for (int i = 0; i < 4; ++i) wreg[i] = 0x88888888u;  // columns past the layout: zero weights
        sc = 1.0f;
        zsc = 8.0f;
      }
    };
    fetch(0);
    for (int kc = 0; kc < w.k; kc += kBK) {
      __syncthreads();  // the previous step's MFMAs are done with the LDS tiles
#pragma unroll
      for (int i = 0; i < 4; ++i) *reinterpret_cast<uint4*>(&xs[xr * kLd + xh + 8 * i]) = xreg[i];
#pragma unroll
      for (int i = 0; i < 4; ++i)
        *reinterpret_cast<uint4*>(&wsm[wc * kLd + (wr0 + i) * 8]) = dequant_word(wreg[i], sc, zsc);
      __syncthreads();
      if (kc + kBK < w.k) fetch(kc + kBK);
#pragma unroll
      for (int k16 = 0; k16 < kBK / 16; ++k16) {
        const int kk = k16 * 16 + (lane >> 5) * 8;
        uint4 a[2], b[2];
#pragma unroll
        for (int mb = 0; mb < 2; ++mb)
          a[mb] = *reinterpret_cast<const uint4*>(&xs[(wm * 64 + mb * 32 + (lane & 31)) * kLd + kk]);
#pragma unroll
        for (int nb = 0; nb < 2; ++nb)
          b[nb] = *reinterpret_cast<const uint4*>(&wsm[(wn * 64 + nb * 32 + (lane & 31)) * kLd + kk]);
#pragma unroll
        for (int mb = 0; mb < 2; ++mb)
#pragma unroll
          for (int nb = 0; nb < 2; ++nb) acc[mb][nb] = mfma32(a[mb], b[nb], acc[mb][nb]);
      }
    }
  }

  const int64_t prow = p0 + wm * 64;
  const int pcol = n0 + wn * 64;
  int32_t orig[2][16];  // original token index of each accumulator row (-1 past the tokens)
#pragma unroll
  for (int mb = 0; mb < 2; ++mb)
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int64_t p = prow + mb * 32 + (i >> 2) * 8 + (lane >> 5) * 4 + (i & 3);
      orig[mb][i] = p < T ? r.tok_perm[p] : -1;
    }
  if constexpr (!kBase) {  // lora_add: start from y
#pragma unroll
    for (int mb = 0; mb < 2; ++mb)
#pragma unroll
      for (int nb = 0; nb < 2; ++nb) {
        const int c = pcol + nb * 32 + (lane & 31);
#pragma unroll
        for (int i = 0; i < 16; ++i)
          if (orig[mb][i] >= 0 && c < n_out) acc[mb][nb][i] = bf16_to_f32(y[(int64_t)orig[mb][i] * y_stride + c]);
      }
  }
  expand_into(acc, prow, pcol, L, r, mid, n_out, lane);
#pragma unroll
  for (int mb = 0; mb < 2; ++mb)
#pragma unroll
    for (int nb = 0; nb < 2; ++nb) {
      const int c = pcol + nb * 32 + (lane & 31);
      if (c >= n_out) continue;
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        if (orig[mb][i] < 0) continue;
        const uint16_t v = f32_to_bf16(acc[mb][nb][i]);
        y[(int64_t)orig[mb][i] * y_stride + c] = v;
        if (last_out != nullptr) {
          const int64_t p = prow + mb * 32 + (i >> 2) * 8 + (lane >> 5) * 4 + (i & 3);
          const int q = r.last_of[p];
          if (q >= 0) last_out[(int64_t)q * n_out + c] = v;
        }
      }
    }
}

constexpr int kGvCols = 16, kGvSlices = 64;  // columns per workgroup; input slices (4 columns x 64 slices = 256 threads)
constexpr int kGvMaxTokens = 8;
constexpr int kGvChunk = 2048;               // inputs of x staged in LDS at a time (8 rows x 4 KB)
constexpr int kGvRows = kGvChunk / 8 / kGvSlices;  // word rows per thread and chunk
constexpr int kBigTileTokens = 1024;  // from here on the 256 x 256 tiles of gemm256.hip fill the chip

static_assert(kGvSlices * kGvMaxTokens * kGvCols * 4 <= kGvMaxTokens * kGvChunk * 2, "the sums reuse the x buffer");

// At most 8 tokens. A workgroup takes 16 columns: thread (slice ks, column group cg) the 4 columns 4 cg .. +3 and the
// word rows ks, ks + 64, ... of each 2048-input chunk. Per chunk, every thread first issues all its loads (the words
// of its rows, their scales and zero points) and the workgroup stages the chunk of the 8 token rows of x in LDS
// (loads that write LDS directly), then waits once; each word is dequantised once and dotted with every token
// (v_dot2_f32_bf16). The 64 slices' sums are added in slice order through LDS (the x buffer's space), then each
// output adds its LoRA term (eight ranks per 16-byte load) and is rounded once. Without the base (kBase = false) the
// output adds the LoRA term to y in place (lora_add).
template <bool kBase>
__global__ __launch_bounds__(256) void base_gemv_kernel(mlora_int4_t w, mlora_lora_t L, mlora_route_t r,
                                                       const uint16_t* __restrict__ x, int64_t x_stride,
                                                       uint16_t* __restrict__ y, int64_t y_stride,
                                                       uint16_t* __restrict__ last_out, int32_t n_out,
                                                       const uint16_t* __restrict__ mid) {
  __shared__ __attribute__((aligned(16))) uint16_t xs[kGvMaxTokens * kGvChunk];
  float* red = reinterpret_cast<float*>(xs);  // [slice][token][column], after the last chunk
  const int tid = threadIdx.x;
  const int n0 = blockIdx.x * kGvCols;
  const int T = (int)r.tokens;
  if constexpr (kBase) {
    const int cg = tid & 3, ks = tid >> 2;
    const int c4 = n0 + cg * 4;  // columns is a multiple of 64: c4 + 3 < columns
    const bool vec_sz = (reinterpret_cast<uintptr_t>(w.scales) & 7) == 0 &&
                        (w.zeros == nullptr || (reinterpret_cast<uintptr_t>(w.zeros) & 3) == 0);
    // x staging: instruction i of thread t moves 16 bytes: token row (256 i + t) / 256, 16-byte column (256 i + t)
    // % 256 of the chunk (rows past the tokens read the last token's row; their sums are never written)
    const uint16_t* xrow[kGvMaxTokens];
#pragma unroll
    for (int m = 0; m < kGvMaxTokens; ++m) xrow[m] = x + (int64_t)r.tok_perm[min(m, T - 1)] * x_stride;
    float acc[kGvMaxTokens][4];
#pragma unroll
    for (int m = 0; m < kGvMaxTokens; ++m)
#pragma unroll
      for (int e = 0; e < 4; ++e) acc[m][e] = 0.0f;
    for (int k0 = 0; k0 < w.k; k0 += kGvChunk) {
      const int kn = min(kGvChunk, w.k - k0);  // a multiple of 64
      // the thread's word rows of this chunk, their scales and zero points
      uint4 wv[kGvRows];
      uint32_t sb[kGvRows][4], zb[kGvRows][4];
#pragma unroll
      for (int i = 0; i < kGvRows; ++i) {
        const int wr = (k0 + 8 * (ks + kGvSlices * i)) / 8;
        const bool in = 8 * (ks + kGvSlices * i) < kn;
        const int wrc = in ? wr : k0 / 8;  // rows past the chunk re-read its first (their products are not added)
        const int64_t g = (int64_t)((8 * wrc) / w.group) * w.columns + c4;
        wv[i] = *reinterpret_cast<const uint4*>(w.words + (int64_t)wrc * w.columns + c4);
        if (vec_sz) {
          const uint2 sv = *reinterpret_cast<const uint2*>(w.scales + g);
          const uint32_t zv = w.zeros != nullptr ? *reinterpret_cast<const uint32_t*>(w.zeros + g) : 0x08080808u;
          sb[i][0] = sv.x & 0xFFFF, sb[i][1] = sv.x >> 16, sb[i][2] = sv.y & 0xFFFF, sb[i][3] = sv.y >> 16;
#pragma unroll
          for (int e = 0; e < 4; ++e) zb[i][e] = (zv >> (8 * e)) & 0xFF;
        } else {
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            sb[i][e] = w.scales[g + e];
            zb[i][e] = w.zeros != nullptr ? w.zeros[g + e] : 8;
          }
        }
      }
      __syncthreads();  // the previous chunk's x reads are done
#pragma unroll
      for (int i = 0; i < kGvMaxTokens; ++i) {
        const int e = 256 * i + tid, m = e >> 8, c16 = e & 255;
        if (8 * c16 < kn)
          __builtin_amdgcn_global_load_lds(xrow[m] + k0 + 8 * c16, (lds_void*)(xs + m * kGvChunk + 8 * c16), 16, 0,
                                           0);
      }
      MLORA_WAIT_VM(0);  // every load of this thread
      __syncthreads();
#pragma unroll
      for (int i = 0; i < kGvRows; ++i) {
        const int kk = 8 * (ks + kGvSlices * i);
        if (kk >= kn) break;
        const uint32_t wd[4] = {wv[i].x, wv[i].y, wv[i].z, wv[i].w};
        uint4 wq[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float sc = bf16_to_f32(sb[i][e]);
          wq[e] = dequant_word(wd[e], sc, (float)zb[i][e] * sc);
        }
#pragma unroll
        for (int m = 0; m < kGvMaxTokens; ++m) {
          const uint4 xv = *reinterpret_cast<const uint4*>(xs + m * kGvChunk + kk);
#pragma unroll
          for (int e = 0; e < 4; ++e) acc[m][e] = dot8(xv, wq[e], acc[m][e]);
        }
      }
    }
    __syncthreads();  // the x buffer becomes the slices' sums
#pragma unroll
    for (int m = 0; m < kGvMaxTokens; ++m)
#pragma unroll
      for (int e = 0; e < 4; ++e) red[(ks * kGvMaxTokens + m) * kGvCols + cg * 4 + e] = acc[m][e];
    __syncthreads();
  }
  // output (token m, column c) of threads 0..127
  const int m = tid / kGvCols, cl = tid % kGvCols;
  const int c = n0 + cl;
  if (tid >= kGvMaxTokens * kGvCols || m >= T || c >= n_out) return;
  const int t = r.tok_perm[m];
  float v;
  if constexpr (kBase) {
    v = 0.0f;
    for (int s = 0; s < kGvSlices; ++s) v += red[(s * kGvMaxTokens + m) * kGvCols + cl];
  } else {
    v = bf16_to_f32(y[(int64_t)t * y_stride + c]);
  }
  const int a = r.seg_adapter[r.seg_of[m]];
  const int j = matrix_of(L, c);
  const int rank = a != 0 ? live_rank(L, a, j) : 0;
  if (rank > 0) {
    const uint16_t* mr = mid + (int64_t)m * L.rank_cap + rank_offset(L, j);
    const uint16_t* br = L.pool + (int64_t)a * L.pool_stride + L.off_b[j] +
                         (int64_t)(c - col_offset(L, j)) * sb_stride(rank, L.cap[j]);
    // eight ranks per 16-byte load of each (rank offsets, capacities and row strides are multiples of 8); the chunk
    // crossing the live rank keeps its live ranks only
    float lora = 0.0f;
    for (int q = 0; q < rank; q += 8) {
      const uint4 mv = keep_first(*reinterpret_cast<const uint4*>(mr + q), rank - q);
      const uint4 bv = keep_first(*reinterpret_cast<const uint4*>(br + q), rank - q);
      lora = dot8(mv, bv, lora);
    }
    v += lora;
  }
  const uint16_t o = f32_to_bf16(v);
  y[(int64_t)t * y_stride + c] = o;
  if (last_out != nullptr && r.last_of[m] >= 0) last_out[(int64_t)r.last_of[m] * n_out + c] = o;
}

}  // namespace

int launch_base(const mlora_int4_t* w, const mlora_lora_t& L, const mlora_route_t& r, const uint16_t* x,
                int64_t x_stride, uint16_t* y, int64_t y_stride, uint16_t* last_out, int32_t n_out,
                const uint16_t* mid, bool gemv, hipStream_t stream) {
  if (r.tokens == 0 || n_out == 0) return MLORA_OK;
  const mlora_int4_t none = {};
  if (gemv) {
    const int blocks = (n_out + kGvCols - 1) / kGvCols;
    if (w != nullptr)
      hipLaunchKernelGGL(base_gemv_kernel<true>, dim3(blocks), dim3(256), 0, stream, *w, L, r, x, x_stride, y,
                         y_stride, last_out, n_out, mid);
    else
      hipLaunchKernelGGL(base_gemv_kernel<false>, dim3(blocks), dim3(256), 0, stream, none, L, r, x, x_stride, y,
                         y_stride, last_out, n_out, mid);
  } else if (w != nullptr && r.tokens >= kBigTileTokens && r.tokens * x_stride < ((int64_t)1 << 31)) {
    // (the 256 x 256 kernel addresses x rows with 32-bit element offsets)
    return launch_base256(*w, L, r, x, x_stride, y, y_stride, last_out, n_out, mid, nullptr, 1, stream);
  } else {
    const int m_tiles = (int)((r.tokens + kBM - 1) / kBM);
    const int n_tiles = (n_out + kBN - 1) / kBN;
    const int64_t blocks = (int64_t)m_tiles * n_tiles;
    if (w != nullptr)
      hipLaunchKernelGGL(base_mfma_kernel<true>, dim3((unsigned)blocks), dim3(256), 0, stream, *w, L, r, x, x_stride,
                         y, y_stride, last_out, n_out, mid, m_tiles);
    else
      hipLaunchKernelGGL(base_mfma_kernel<false>, dim3((unsigned)blocks), dim3(256), 0, stream, none, L, r, x,
                         x_stride, y, y_stride, last_out, n_out, mid, m_tiles);
  }
  return hipGetLastError() == hipSuccess ? MLORA_OK : MLORA_ELAUNCH;
}
