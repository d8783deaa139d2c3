// Prefill-sized INT4 base product with the LoRA second factor fused (the same arithmetic as base.hip's kernels):
//   y[perm[p], c] = bf16( sum_k x[perm[p], k] W[c, k] + sum_q mid[p, rho_j + q] sB_j[a][c - o_j, q] )
// Tiles of 256 sorted tokens x 256 columns, 8 waves of 128 x 64 (2 x 4), 32x32x16 bf16 MFMA, float32 accumulation.
// Each K step of 64 inputs stages the gathered x rows and the dequantised weights through double-buffered LDS
// (2 x 2 x 36 KB): the next step's words and activations are fetched into registers while the MFMAs of the current
// step run, and written to the other buffer afterwards, so one barrier per step suffices. Two waves per SIMD let the
// hardware interleave one wave's dequantisation (VALU) with the other's MFMAs.
// Tiles are ordered so that the column tiles of one row tile run on the same XCD: its x rows (the larger operand)
// are read from HBM once per XCD and then hit that XCD's L2.
// Epilogue: each adapter segment crossing the tile has its sB rows for the tile's 256 columns staged in LDS with
// coalesced 16-byte loads, and added by MFMA with the tokens' first factors (zero outside the segment), before the
// single rounding to bf16.
#include "mlora_common.h"

namespace {

using namespace mlora;

constexpr int kTM = 256, kTN = 256, kTK = 64;
constexpr int kLd = kTK + 8;          // LDS row stride in bf16 (144 bytes): 16-byte reads of 32 rows are conflict-free
constexpr int kBuf = kTM * kLd;       // one staged operand
constexpr int kThreads = 512;
constexpr int kRankChunk = 64;        // ranks of sB staged per epilogue pass

// blockIdx -> tile index such that consecutive tiles share an XCD (blocks are dealt to the 8 XCDs round-robin)
__device__ __forceinline__ int xcd_tile(int b, int nb) {
  const int per = nb / 8, extra = nb % 8;
  const int xcd = b % 8, slot = b / 8;
  return xcd * per + min(xcd, extra) + slot;
}

__global__ __launch_bounds__(kThreads) void base_mfma256_kernel(mlora_int4_t w, mlora_lora_t L, mlora_route_t r,
                                                               const uint16_t* __restrict__ x, int64_t x_stride,
                                                               uint16_t* __restrict__ y, int64_t y_stride,
                                                               uint16_t* __restrict__ last_out, int32_t n_out,
                                                               const uint16_t* __restrict__ mid, int32_t n_tiles) {
  __shared__ __attribute__((aligned(16))) uint16_t lds[4 * kBuf];  // x0, x1, w0, w1
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 2, wn = wave & 3;
  const int t = xcd_tile(blockIdx.x, gridDim.x);
  const int mt = t / n_tiles, nt = t - mt * n_tiles;
  const int64_t T = r.tokens;
  const int64_t p0 = (int64_t)mt * kTM;
  const int n0 = nt * kTN;

  const int xr = tid >> 1, xh = (tid & 1) * 32;  // x staging: 32 inputs of one gathered row
  const int64_t xp = p0 + xr;
  const uint16_t* xsrc = xp < T ? x + (int64_t)r.tok_perm[xp] * x_stride + xh : nullptr;
  const int wc = tid & (kTN - 1), wr0 = (tid >> 8) * 4;  // weight staging: 4 words (32 inputs) of one column
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
  auto stage = [&](int buf) {
    uint16_t* xs = lds + buf * kBuf;
    uint16_t* ws = lds + (2 + buf) * kBuf;
#pragma unroll
    for (int i = 0; i < 4; ++i) *reinterpret_cast<uint4*>(&xs[xr * kLd + xh + 8 * i]) = xreg[i];
#pragma unroll
    for (int i = 0; i < 4; ++i)
      *reinterpret_cast<uint4*>(&ws[wc * kLd + (wr0 + i) * 8]) = dequant_word(wreg[i], sc, zsc);
  };

  f32x16_t acc[4][2];
#pragma unroll
  for (int mb = 0; mb < 4; ++mb)
#pragma unroll
    for (int nb = 0; nb < 2; ++nb) acc[mb][nb] = f32x16_t{};

  const int nk = w.k / kTK;
  fetch(0);
  stage(0);
  if (nk > 1) fetch(kTK);
  __syncthreads();
  for (int it = 0; it < nk; ++it) {
    const uint16_t* xs = lds + (it & 1) * kBuf;
    const uint16_t* ws = lds + (2 + (it & 1)) * kBuf;
#pragma unroll
    for (int k16 = 0; k16 < kTK / 16; ++k16) {
      const int kk = k16 * 16 + (lane >> 5) * 8;
      uint4 a[4], b[2];
#pragma unroll
      for (int mb = 0; mb < 4; ++mb)
        a[mb] = *reinterpret_cast<const uint4*>(&xs[(wm * 128 + mb * 32 + (lane & 31)) * kLd + kk]);
#pragma unroll
      for (int nb = 0; nb < 2; ++nb)
        b[nb] = *reinterpret_cast<const uint4*>(&ws[(wn * 64 + nb * 32 + (lane & 31)) * kLd + kk]);
#pragma unroll
      for (int mb = 0; mb < 4; ++mb)
#pragma unroll
        for (int nb = 0; nb < 2; ++nb) acc[mb][nb] = mfma32(a[mb], b[nb], acc[mb][nb]);
    }
    if (it + 1 < nk) stage((it + 1) & 1);
    if (it + 2 < nk) fetch((it + 2) * kTK);
    __syncthreads();
  }

  // LoRA second factor, one adapter segment at a time
  const int nseg = *r.num_segs;
  const int64_t tile_end = min(p0 + kTM, T);
  uint16_t* bl = lds;  // staged sB rows: [256 columns][kLd], ranks rc..rc+63
  for (int s = segment_of(r.seg_start, nseg, p0); s < nseg && r.seg_start[s] < tile_end; ++s) {
    const int a = r.seg_adapter[s];
    if (a == 0) continue;  // the base row: no update
    const int64_t sb = r.seg_start[s], se = r.seg_start[s + 1];
    int rk[MLORA_MAX_MATS];
    int maxr = 0;
    const int jfirst = matrix_of(L, n0), jlast = matrix_of(L, min(n0 + kTN, n_out) - 1);
    for (int j = 0; j < L.n_mats; ++j) {
      rk[j] = live_rank(L, a, j);
      if (j >= jfirst && j <= jlast) maxr = max(maxr, rk[j]);
    }
    const uint16_t* prow = L.pool + (int64_t)a * L.pool_stride;
    for (int rc = 0; rc < maxr; rc += kRankChunk) {
      const int c = tid & (kTN - 1), half = tid >> 8;
      const int gc = n0 + c;
      uint4 v[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) v[i] = make_uint4(0, 0, 0, 0);
      if (gc < n_out) {
        const int j = matrix_of(L, gc);
        const uint16_t* src = prow + L.off_b[j] + (int64_t)(gc - col_offset(L, j)) * L.cap[j];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int kk = rc + half * 32 + i * 8;
          if (kk < rk[j]) v[i] = keep_first(*reinterpret_cast<const uint4*>(src + kk), rk[j] - kk);
        }
      }
      __syncthreads();  // the previous pass is done with bl
#pragma unroll
      for (int i = 0; i < 4; ++i) *reinterpret_cast<uint4*>(&bl[c * kLd + half * 32 + i * 8]) = v[i];
      __syncthreads();
#pragma unroll
      for (int mb = 0; mb < 4; ++mb) {
        const int64_t r0 = p0 + wm * 128 + mb * 32;
        if (r0 >= se || r0 + 32 <= sb || r0 >= T) continue;
        const int64_t row = r0 + (lane & 31);
        const bool rowok = row >= sb && row < se;
#pragma unroll
        for (int nb = 0; nb < 2; ++nb) {
          const int c0 = n0 + wn * 64 + nb * 32;
          if (c0 >= n_out) continue;
          const int cc = c0 + (lane & 31);
          const int jlo = matrix_of(L, c0), jhi = matrix_of(L, min(c0 + 31, n_out - 1));
          for (int j = jlo; j <= jhi; ++j) {
            const int rj = rk[j];
            if (rj <= rc) continue;
            const int oj = col_offset(L, j);
            const bool colok2 = cc >= oj && cc < oj + L.cols[j] && cc < n_out;
            const uint16_t* mrow = mid + (rowok ? row : 0) * L.rank_cap + rank_offset(L, j);
            const int kend = min(rj, rc + kRankChunk);
            for (int k0 = rc; k0 < kend; k0 += 16) {
              const int kk = k0 + (lane >> 5) * 8;
              const int nvalid = rj - kk;
              uint4 av = make_uint4(0, 0, 0, 0), bv = av;
              if (nvalid > 0) {
                if (rowok) av = keep_first(*reinterpret_cast<const uint4*>(mrow + kk), nvalid);
                if (colok2) bv = *reinterpret_cast<const uint4*>(&bl[(cc - n0) * kLd + (kk - rc)]);
              }
              acc[mb][nb] = mfma32(av, bv, acc[mb][nb]);
            }
          }
        }
      }
    }
  }

#pragma unroll
  for (int mb = 0; mb < 4; ++mb) {
    int32_t orig[16], lastq[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int64_t p = p0 + wm * 128 + mb * 32 + (i >> 2) * 8 + (lane >> 5) * 4 + (i & 3);
      orig[i] = p < T ? r.tok_perm[p] : -1;
      lastq[i] = (p < T && last_out != nullptr) ? r.last_of[p] : -1;
    }
#pragma unroll
    for (int nb = 0; nb < 2; ++nb) {
      const int c = n0 + wn * 64 + nb * 32 + (lane & 31);
      if (c >= n_out) continue;
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        if (orig[i] < 0) continue;
        const uint16_t v = f32_to_bf16(acc[mb][nb][i]);
        y[(int64_t)orig[i] * y_stride + c] = v;
        if (lastq[i] >= 0) last_out[(int64_t)lastq[i] * n_out + c] = v;
      }
    }
  }
}

}  // namespace

int launch_base256(const mlora_int4_t& w, const mlora_lora_t& L, const mlora_route_t& r, const uint16_t* x,
                   int64_t x_stride, uint16_t* y, int64_t y_stride, uint16_t* last_out, int32_t n_out,
                   const uint16_t* mid, hipStream_t stream) {
  if (r.tokens == 0 || n_out == 0) return MLORA_OK;
  const int m_tiles = (int)((r.tokens + kTM - 1) / kTM);
  const int n_tiles = (n_out + kTN - 1) / kTN;
  const int64_t blocks = (int64_t)m_tiles * n_tiles;
  hipLaunchKernelGGL(base_mfma256_kernel, dim3((unsigned)blocks), dim3(kThreads), 0, stream, w, L, r, x, x_stride, y,
                     y_stride, last_out, n_out, mid, n_tiles);
  return hipGetLastError() == hipSuccess ? MLORA_OK : MLORA_ELAUNCH;
}
