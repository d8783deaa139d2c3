// Prefill-sized INT4 base product with the LoRA second factor fused (the same arithmetic as base.hip's kernels):
//   y[perm[p], c] = bf16( sum_k x[perm[p], k] W[c, k] + sum_q mid[p, rho_j + q] sB_j[a][c - o_j, q] )
// Tiles of 256 sorted tokens x 256 columns, 8 waves of 128 x 64 (2 x 4), 32x32x16 bf16 MFMA, float32 accumulators;
// two waves per SIMD.
//
// Per K step of 64 inputs:
//  - x: the 256 gathered rows go straight from memory to LDS with global_load_lds (16 bytes per lane, no registers),
//    two steps ahead, into a ring of three LDS buffers; the waves read their A operands from it;
//  - weights: no LDS at all. Each lane loads the packed words that form its own B operands (one 32-bit word = the 8
//    consecutive inputs of one column that a 32x32x16 operand lane holds), one step ahead, with the raw scale and
//    zero point of its columns, and dequantises them to bf16((c - z) s) in registers right before the MFMAs. The two
//    waves sharing a column range both dequantise it, which costs VALU time that their MFMAs hide.
// With no LDS stores in the loop, nothing but the x ring is ordered by the step barrier: a plain s_barrier after an
// explicit wait for the x rows of the next step (a __syncthreads() would also wait for the rows two steps ahead).
// LDS rows are 128 bytes (64 bf16) with their eight 16-byte chunks XOR-swizzled by (row & 7): the 16-byte A-operand
// reads of 8 consecutive rows hit 8 distinct chunk positions, i.e. all banks once. The ring buffers are distinct LDS
// arrays chosen at compile time (the loop is unrolled by three). Tiles are ordered so that the column tiles of one
// row tile run on the same XCD (its x rows, the larger operand, then come from that XCD's L2).
// Epilogue: each adapter segment crossing the tile has its sB rows for the tile's 256 columns staged in LDS with
// coalesced 16-byte loads and added by MFMA with the tokens' first factors (zero outside the segment), then the
// single rounding to bf16.
#include <type_traits>

#include "mlora_common.h"

namespace {

using namespace mlora;

constexpr int kTM = 256, kTN = 256, kTK = 64;
constexpr int kThreads = 512;
constexpr int kRankChunk = 64;   // ranks of sB staged per epilogue pass
constexpr int kXLoads = 4;       // global_load_lds instructions per lane and step
constexpr int kWLoads = 8 + 4;   // weight loads per lane and step: 2 x 4 words, 2 scales, 2 zero points

typedef __attribute__((address_space(3))) void lds_void;

__shared__ __attribute__((aligned(16))) uint16_t g_x0[kTM * kTK];
__shared__ __attribute__((aligned(16))) uint16_t g_x1[kTM * kTK];
__shared__ __attribute__((aligned(16))) uint16_t g_x2[kTM * kTK];

// Element offset of 16-byte chunk c of row `row` in a swizzled 64-element-per-row tile.
__device__ __forceinline__ int swz(int row, int c) { return row * kTK + ((c ^ (row & 7)) << 3); }

// Wait until at most n vector memory instructions of this wave are outstanding and its LDS operations are done
// (gfx9 s_waitcnt encoding: vmcnt in bits 3:0 and 15:14, expcnt 6:4 left at its maximum, lgkmcnt 11:8 = 0).
#define MLORA_WAIT_VM(n) __builtin_amdgcn_s_waitcnt(((n) & 0xF) | (((n) >> 4) << 14) | (0x7 << 4))

// blockIdx -> tile index such that consecutive tiles share an XCD (blocks are dealt to the 8 XCDs round-robin)
__device__ __forceinline__ int xcd_tile(int b, int nb) {
  const int per = nb / 8, extra = nb % 8;
  const int xcd = b % 8, slot = b / 8;
  return xcd * per + min(xcd, extra) + slot;
}

// One step's weights as loaded by a lane: word [nb][k16] of each of its two 32-column blocks, and the raw bf16
// scale and zero point of its two columns (converted only when used, a step later)
struct WStage {
  uint32_t w[2][4];
  uint32_t sbits[2], zbyte[2];
};

__global__ __launch_bounds__(kThreads) void base_mfma256_kernel(mlora_int4_t w, mlora_lora_t L, mlora_route_t r,
                                                               const uint16_t* __restrict__ x, int64_t x_stride,
                                                               uint16_t* __restrict__ y, int64_t y_stride,
                                                               uint16_t* __restrict__ last_out, int32_t n_out,
                                                               const uint16_t* __restrict__ mid, int32_t n_tiles) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 2, wn = wave & 3;
  const int t = xcd_tile(blockIdx.x, gridDim.x);
  const int mt = t / n_tiles, nt = t - mt * n_tiles;
  const int64_t T = r.tokens;
  const int64_t p0 = (int64_t)mt * kTM;
  const int n0 = nt * kTN;

  // Loads go through buffer resources: the per-lane byte offsets below stay fixed for the whole K loop and the K
  // position is a wave-uniform scalar offset, so no 64-bit addresses are kept in registers. The resources' sizes
  // are the arrays' sizes (the host keeps tokens x x_stride below 2^31 elements).
  const __amdgpu_buffer_rsrc_t xres =
      __builtin_amdgcn_make_buffer_rsrc((void*)x, (short)0, 0x7fffffff, 0x00020000);
  const __amdgpu_buffer_rsrc_t wres = __builtin_amdgcn_make_buffer_rsrc(
      (void*)w.words, (short)0, (int)((int64_t)(w.k / 8) * w.columns * 4), 0x00020000);
  const int64_t groups = w.k / w.group;
  const __amdgpu_buffer_rsrc_t sres = __builtin_amdgcn_make_buffer_rsrc(
      (void*)w.scales, (short)0, (int)(groups * w.columns * 2), 0x00020000);
  const bool asym = w.zeros != nullptr;
  const __amdgpu_buffer_rsrc_t zres = __builtin_amdgcn_make_buffer_rsrc(
      asym ? (void*)w.zeros : (void*)w.scales, (short)0, (int)(groups * w.columns), 0x00020000);

  // x: instruction i of wave `wave` fills rows (8 i + wave) * 8 .. +7; lane l writes LDS chunk slot l & 7 of row
  // +(l >> 3), which holds logical chunk (l & 7) ^ (l >> 3). Rows past the tokens read row 0 of the pass.
  uint32_t xoff[kXLoads];
#pragma unroll
  for (int i = 0; i < kXLoads; ++i) {
    const int row = (8 * i + wave) * 8 + (lane >> 3);
    const int64_t p = p0 + row;
    xoff[i] = (uint32_t)(((int64_t)r.tok_perm[p < T ? p : 0] * x_stride + (((lane & 7) ^ (lane >> 3)) << 3)) * 2);
  }
  auto dma_x = [&](uint16_t* buf, int kc) {
#pragma unroll
    for (int i = 0; i < kXLoads; ++i)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(xres, (lds_void*)(buf + (8 * i + wave) * 8 * kTK), 16, xoff[i], kc * 2,
                                               0, 0);
  };

  // weights: lane l of block nb holds column n0 + 64 wn + 32 nb + (l & 31) and, for 16 inputs k16, the word of
  // inputs 16 k16 + 8 (l >> 5) .. +7; columns past the layout read column 0 and get zero weights (scale 0)
  bool colok[2];
  uint32_t woff[2], soff[2], zoff[2];
#pragma unroll
  for (int nb = 0; nb < 2; ++nb) {
    const int c = n0 + wn * 64 + nb * 32 + (lane & 31);
    colok[nb] = c < w.columns;
    const uint32_t gc = colok[nb] ? c : 0;
    woff[nb] = (gc + (uint32_t)(lane >> 5) * w.columns) * 4;
    soff[nb] = gc * 2;
    zoff[nb] = asym ? gc : gc * 2;
  }
  const int wstep = w.columns * 8;  // bytes between the words of k16 and k16 + 1
  auto fetch_w = [&](WStage& st, int kc) {
    const int wbase = (kc / 8) * w.columns * 4;
#pragma unroll
    for (int nb = 0; nb < 2; ++nb)
#pragma unroll
      for (int k16 = 0; k16 < 4; ++k16)
        st.w[nb][k16] = __builtin_amdgcn_raw_buffer_load_b32(wres, woff[nb], wbase + k16 * wstep, 0);
    const int g = (kc / w.group) * w.columns;
#pragma unroll
    for (int nb = 0; nb < 2; ++nb) {
      st.sbits[nb] = __builtin_amdgcn_raw_buffer_load_b16(sres, soff[nb], g * 2, 0);
      st.zbyte[nb] = __builtin_amdgcn_raw_buffer_load_b8(zres, zoff[nb], asym ? g : g * 2, 0);
    }
  };

  f32x16_t acc[4][2];
#pragma unroll
  for (int mb = 0; mb < 4; ++mb)
#pragma unroll
    for (int nb = 0; nb < 2; ++nb) acc[mb][nb] = f32x16_t{};

  auto load_a = [&](const uint16_t* xs, int k16, uint4 (&a)[4]) {
    const int c = 2 * k16 + (lane >> 5);
#pragma unroll
    for (int mb = 0; mb < 4; ++mb)
      a[mb] = *reinterpret_cast<const uint4*>(&xs[swz(wm * 128 + mb * 32 + (lane & 31), c)]);
  };
  // one K step: A operands from the x buffer (the next 16 inputs' read while the current ones are multiplied), B
  // operands dequantised in registers from the step's words
  auto step = [&](const uint16_t* xs, const WStage& ws) {
    float sv[2], zs[2];
#pragma unroll
    for (int nb = 0; nb < 2; ++nb) {
      const float s0v = bf16_to_f32(ws.sbits[nb]);
      const float zv = asym ? (float)ws.zbyte[nb] : 8.0f;
      sv[nb] = colok[nb] ? s0v : 0.0f;
      zs[nb] = colok[nb] ? zv * s0v : 0.0f;
    }
    uint4 a0[4], a1[4];
    load_a(xs, 0, a0);
#pragma unroll
    for (int k16 = 0; k16 < kTK / 16; ++k16) {
      uint4 (&ca)[4] = (k16 & 1) ? a1 : a0;
      uint4 (&na)[4] = (k16 & 1) ? a0 : a1;
      if (k16 + 1 < kTK / 16) load_a(xs, k16 + 1, na);
      uint4 b[2];
#pragma unroll
      for (int nb = 0; nb < 2; ++nb) b[nb] = dequant_word(ws.w[nb][k16], sv[nb], zs[nb]);
#pragma unroll
      for (int mb = 0; mb < 4; ++mb)
#pragma unroll
        for (int nb = 0; nb < 2; ++nb) acc[mb][nb] = mfma32(ca[mb], b[nb], acc[mb][nb]);
    }
  };

  // Step i reads x buffer i % 3 (its rows loaded at the start of step i - 2) and weight set i % 2 (loaded at the
  // start of step i - 1). Every load is unconditional (past the last step it re-reads the last one into a buffer or
  // set that is never used), so the number of loads in flight at each wait is the same on every path:
  // after x(i + 1) come w(i), x(i + 2) and w(i + 1).
  const int nk = w.k / kTK;
  WStage s0, s1;
  dma_x(g_x0, 0);
  fetch_w(s0, 0);
  dma_x(g_x1, min(1, nk - 1) * kTK);
  MLORA_WAIT_VM(kWLoads + kXLoads);  // x(0) has landed
  __builtin_amdgcn_s_barrier();
  auto run = [&](auto xb, auto wb, int i) {
    constexpr int XB = decltype(xb)::value, WB = decltype(wb)::value;
    const uint16_t* xs = XB == 0 ? g_x0 : XB == 1 ? g_x1 : g_x2;
    uint16_t* xf = XB == 0 ? g_x2 : XB == 1 ? g_x0 : g_x1;  // buffer (i + 2) % 3
    WStage& cur = WB == 0 ? s0 : s1;
    WStage& nxt = WB == 0 ? s1 : s0;
    dma_x(xf, min(i + 2, nk - 1) * kTK);
    fetch_w(nxt, min(i + 1, nk - 1) * kTK);
    step(xs, cur);
    MLORA_WAIT_VM(kWLoads + kXLoads + kWLoads);  // x(i + 1) has landed
    __builtin_amdgcn_s_barrier();
  };
  using I0 = std::integral_constant<int, 0>;
  using I1 = std::integral_constant<int, 1>;
  using I2 = std::integral_constant<int, 2>;
  for (int it = 0; it < nk; it += 6) {
    run(I0{}, I0{}, it);
    if (it + 1 >= nk) break;
    run(I1{}, I1{}, it + 1);
    if (it + 2 >= nk) break;
    run(I2{}, I0{}, it + 2);
    if (it + 3 >= nk) break;
    run(I0{}, I1{}, it + 3);
    if (it + 4 >= nk) break;
    run(I1{}, I0{}, it + 4);
    if (it + 5 >= nk) break;
    run(I2{}, I1{}, it + 5);
  }
  MLORA_WAIT_VM(0);
  __builtin_amdgcn_s_barrier();

  // LoRA second factor, one adapter segment at a time; sB rows are staged in g_x0 (swizzled like x)
  const int nseg = *r.num_segs;
  const int64_t tile_end = min(p0 + kTM, T);
  uint16_t* bl = g_x0;
  const int wcol = tid & (kTN - 1), wh = tid >> 8;
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
      const int gc = n0 + wcol;  // ranks rc + 32 h .. +31 of one column per thread
      uint4 v[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) v[i] = make_uint4(0, 0, 0, 0);
      if (gc < n_out) {
        const int j = matrix_of(L, gc);
        const uint16_t* src = prow + L.off_b[j] + (int64_t)(gc - col_offset(L, j)) * L.cap[j];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int kk = rc + (4 * wh + i) * 8;
          if (kk < rk[j]) v[i] = keep_first(*reinterpret_cast<const uint4*>(src + kk), rk[j] - kk);
        }
      }
      __syncthreads();  // the previous pass (or the main loop) is done with bl
#pragma unroll
      for (int i = 0; i < 4; ++i) *reinterpret_cast<uint4*>(&bl[swz(wcol, 4 * wh + i)]) = v[i];
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
                if (colok2) bv = *reinterpret_cast<const uint4*>(&bl[swz(cc - n0, (kk - rc) >> 3)]);
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
