// Decode-sized INT4 product (every token of the pass in one row tile, at most 256, few tokens per adapter segment):
//   y[perm[p], c] = bf16( sum_k x[perm[p], k] W[c, k] + sum_q mid[p, rho_j + q] sB_j[a(p)][c - o_j, q] )
// The same arithmetic as the prefill kernel (gemm256.hip), tiled for few rows: a tile is all of the pass's sorted
// rows x 64 columns, so a product spreads over the CUs with few or no splits of the input dimension (a 12288-column
// product runs as 192 workgroups over all 2048 inputs). 8 waves in 4 row groups x 2 column groups: a wave owns 64
// rows x 32 columns (two 32x32 MFMA blocks). A step's packed words are loaded and dequantised once for the
// workgroup (one word per thread) into a ring of LDS buffers that every wave reads its weight operands from, and
// each wave reads its 64 rows of x from an LDS ring that buffer loads with the LDS flag fill, as in the prefill kernel;
// words and x rows are loaded three steps ahead, the step's barrier sits in its middle, so the operand reads of each
// half of a step overlap the other half's MFMAs, and a step's words are dequantised two steps ahead, past a barrier.
// One input range (the columns alone fill the CUs): the first factors are computed first (shrink_seg.h, their own
// launch), and the tile adds the LoRA term after its K loop: the first factors of the wave's rows (64 ranks of matrix
// j) are loaded before the loop; the adapter segments crossing those rows are listed one per lane (adapter, live
// rank), and each segment's sB rows (the wave's 32 columns) are staged in an LDS slot of the wave's own (the x ring
// is idle by then) by loads that write LDS directly, whole 128-byte rows, one segment ahead of its MFMAs (the expand
// launch below stages them the same way). A segment's term goes into the row blocks it crosses, with the first factors of rows outside the segment, and ranks past its live rank, set to
// zero. The tile is rounded once and written (plain, added to the residual, or silu(gate) * up).
// S input ranges (the columns alone are too few for the CUs): two launches, neither waiting for another workgroup.
// The first is the ranges' base tiles, each writing its float32 tile in the accumulators' own order (one coalesced
// 1 KB store per MFMA block and column group), and, in the workgroups past them, the first factors (one workgroup per
// (segment, 32-rank block), which read only x and A and so run beside the base tiles: their latency chain overlaps
// the K loops instead of preceding them). The second, dec_expand_kernel, adds the ranges in order and the LoRA term
// per (64-row group, column tile), then rounds once and writes.
#include <type_traits>

#include "shrink_seg.h"
#include "tile_common.h"

namespace {

using namespace mlora;
typedef float f32x4_t __attribute__((ext_vector_type(4)));  // (the non-temporal builtins' operand type)

constexpr int kDThreads = 512;
constexpr int kDRows = 256;               // rows of the tile: every token of the pass
constexpr int kDCG = 2;                   // column groups of 32 (tile of 64 columns)
constexpr int kDRG = 8 / kDCG;            // row groups
constexpr int kDMB = kDRows / kDRG / 32;  // 32-row MFMA blocks per wave
constexpr int kDCols = 32 * kDCG;
constexpr int kDXLoads = 4;               // x rows: LDS-flag buffer loads per lane and step
constexpr int kDWLoads = 3;               // weights: a word, a scale and a zero point per thread and step
constexpr int kDRankChunk = 64;           // ranks of a matrix per LoRA pass
constexpr int kDMaxRanges = 8;            // input ranges of a narrow product (the host allows 1, 2, 4 or 8)
constexpr int kESG = 4;                   // the expand launch: segment groups of a row group's segments
constexpr int kEThreads = 64 * kDCG * kESG;  // one wave per (column group, segment group)

static_assert(kDRows / kDRG == 32 * kDMB, "row groups must cover the tile");
static_assert(kDThreads == kDWaves * 64, "a first-factor workgroup is a base workgroup's threads");
static_assert(kDRows * kTK == kSegLds / 2, "a first-factor workgroup stages A in the first two x buffers");

__shared__ __attribute__((aligned(16))) uint16_t d_x0[kDRows * kTK];
__shared__ __attribute__((aligned(16))) uint16_t d_x1[kDRows * kTK];
__shared__ __attribute__((aligned(16))) uint16_t d_x2[kDRows * kTK];
__shared__ __attribute__((aligned(16))) uint16_t d_x3[kDRows * kTK];
__shared__ uint4 d_w0[8 * kDCols];  // a step's weights, dequantised: 8 input octets x 64 columns of 8 bf16
__shared__ uint4 d_w1[8 * kDCols];
__shared__ uint4 d_w2[8 * kDCols];
__shared__ int32_t d_orig[kDRows];  // the tile's rows: original token index, -1 past the tokens
__shared__ int32_t d_last[kDRows];  // the tile's rows: request whose last token it is, else -1

// Float4 index of (range ks, column tile nt, wave, block mb, column group g, lane) in the partial tiles.
__device__ __forceinline__ int64_t part_index(int ks, int n_tiles, int nt, int wave, int mb, int g, int lane) {
  return ((((int64_t)ks * n_tiles + nt) * 8 + wave) * kDMB * 4 + mb * 4 + g) * 64 + lane;
}

// Steps it + B, it + B + 1, ... of a K loop unrolled by 12 (the period of its 4 x buffers and 3 weight buffers), as
// far as step nk - 1: nested conditions, one exit (a chain of breaks out of the unrolled body compiles to more than the
// register budget of this kernel).
template <int B, class F>
__device__ __forceinline__ void steps_from(F& run, int it, int nk) {
  run(std::integral_constant<int, B>{}, it + B);
  if constexpr (B + 1 < 12) {
    if (it + B + 1 < nk) steps_from<B + 1>(run, it, nk);
  }
}

// GATED: the gated epilogue (silu(gate) * up, inter columns), a template parameter so the plain kernel carries none
// of it. RANGES false: one range, the LoRA term from mid, the output written. RANGES true: each range's tile goes to
// part (no LoRA term, no output), and the blocks past the n_tiles x ksplit tiles (the grid's rest) compute the first
// factors into mid (the tiles come first: they take their CUs at once, and the first-factor blocks, whose LDS share
// is the tiles' share, fill the remaining CUs); a template parameter so that neither form carries the other's code.
template <bool GATED, bool RANGES>
__global__ __launch_bounds__(kDThreads) void dec_kernel(mlora_int4_t w, mlora_lora_t L, mlora_route_t r,
                                                        const uint16_t* x, int64_t x_stride,
                                                        uint16_t* __restrict__ y, int64_t y_stride,
                                                        uint16_t* __restrict__ last_out, int32_t n_out,
                                                        uint16_t* mid, int32_t n_tiles, int32_t vec,
                                                        float4* __restrict__ part, int32_t ksplit, int32_t inter,
                                                        int32_t max_blocks) {
  if constexpr (RANGES) {
    const int sb = (int)blockIdx.x - n_tiles * ksplit;  // a first-factor block: one of max_segs x max_blocks
    if (sb >= 0) {
      shrink_seg_block(L, r, x, x_stride, w.k, mid, max_blocks, sb, d_x0, d_x1);
      return;
    }
  }
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform: LDS addresses of the x loads in SGPRs
  const int cg = wave % kDCG, rg = wave / kDCG;
  // block -> (input range ks, column tile nt), column tiles innermost: blocks of one range (the same x) share an XCD
  const int blocks = n_tiles * ksplit;
  const int b = xcd_tile(blockIdx.x, blocks);
  const int ks = b / n_tiles, nt = b - ks * n_tiles;
  const int T = (int)r.tokens;
  const int n0 = nt * kDCols;
  const int R0 = rg * 32 * kDMB;  // the wave's first row

  const __amdgpu_buffer_rsrc_t xres =
      __builtin_amdgcn_make_buffer_rsrc((void*)x, (short)0, (int)0xFFFFFFFFu, 0x00020000);
  const __amdgpu_buffer_rsrc_t wres = __builtin_amdgcn_make_buffer_rsrc(
      (void*)w.words, (short)0, (int)((int64_t)(w.k / 8) * w.columns * 4), 0x00020000);
  const int64_t groups = w.k / w.group;
  const int gshift = w.group == 128 ? 7 : 6;  // the host accepts groups of 64 and 128 inputs
  const __amdgpu_buffer_rsrc_t sres = __builtin_amdgcn_make_buffer_rsrc(
      (void*)w.scales, (short)0, (int)(groups * w.columns * 2), 0x00020000);
  const bool asym = w.zeros != nullptr;
  const __amdgpu_buffer_rsrc_t zres = __builtin_amdgcn_make_buffer_rsrc(
      asym ? (void*)w.zeros : (void*)w.scales, (short)0, (int)(groups * w.columns), 0x00020000);

  if (tid < kDRows) {
    const bool mine = tid < T;
    d_orig[tid] = mine ? r.tok_perm[tid] : -1;
    d_last[tid] = (mine && last_out != nullptr) ? r.last_of[tid] : -1;
  }
  // x: instruction i of wave `wave` fills rows (8 i + wave) * 8 .. +7; lane l writes LDS chunk slot l & 7 of row
  // +(l >> 3), which holds logical chunk swz_slot(row, l & 7). Rows past the tokens read row 0 of the pass.
  uint32_t xoff[kDXLoads];
#pragma unroll
  for (int i = 0; i < kDXLoads; ++i) {
    const int row = (8 * i + wave) * 8 + (lane >> 3);
    xoff[i] = (uint32_t)(((int64_t)r.tok_perm[row < T ? row : 0] * x_stride + (swz_slot(row, lane & 7) << 3)) * 2);
  }
  auto dma_x = [&](uint16_t* buf, int kc) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < kDXLoads; ++i)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(xres, (lds_void*)(buf + (8 * i + wave) * 8 * kTK), 16, xoff[i], kc * 2,
                                               0, 0);
  };

  // weights: thread t loads word t / 64 of the step (inputs 8 (t / 64) .. +7) of column n0 + t % 64 with that
  // column's raw scale and zero point, and dequantises it once for the whole workgroup into the step's LDS buffer, at
  // 16-byte chunk t, where the MFMA operand of (column, inputs) reads it; columns past the layout read column 0 and
  // get zero weights (scale 0)
  // gated (inter > 0): the tile's first 32 columns are gate columns 32 nt .. +31, its last 32 the same up columns
  const int wcol = GATED ? ((tid & 32) ? inter : 0) + nt * 32 + (tid & 31) : n0 + (tid & (kDCols - 1));
  const bool colok = wcol < w.columns;
  const uint32_t gcol = colok ? wcol : 0;
  const uint32_t woff = (gcol + (uint32_t)(tid / kDCols) * w.columns) * 4;
  const uint32_t soff = gcol * 2;
  const uint32_t zoff = asym ? gcol : gcol * 2;
  auto fetch_w = [&](WStage& st, int kc) __attribute__((always_inline)) {
    st.w[0] = __builtin_amdgcn_raw_buffer_load_b32(wres, woff, (kc / 8) * w.columns * 4, 0);
    const int g = (kc >> gshift) * w.columns;
    st.sbits = __builtin_amdgcn_raw_buffer_load_b16(sres, soff, g * 2, 0);
    st.zbyte = __builtin_amdgcn_raw_buffer_load_b8(zres, zoff, asym ? g : g * 2, 0);
  };
  auto dequant_to = [&](uint4* wb, const WStage& st) __attribute__((always_inline)) {
    const float s0v = bf16_to_f32(st.sbits);
    const float zv = asym ? (float)st.zbyte : 8.0f;
    wb[tid] = dequant_word(st.w[0], colok ? s0v : 0.0f, colok ? zv * s0v : 0.0f);
  };

  f32x16_t acc[kDMB];
#pragma unroll
  for (int mb = 0; mb < kDMB; ++mb) acc[mb] = f32x16_t{};

  // first factors of the wave's rows R0 + 32 mb + (lane & 31), ranks rc + 16 k16 + 8 (lane >> 5) .. +7 of matrix j
  // (zero past the pass's rows and past cap_j)
  auto load_mid = [&](uint4 (&m)[kDMB][4], int j, int rc) __attribute__((always_inline)) {
    const int capj = L.cap[j], rho = rank_offset(L, j);
    const int rows = min(R0 + 32 * kDMB, T);
#pragma unroll
    for (int mb = 0; mb < kDMB; ++mb)
#pragma unroll
      for (int k16 = 0; k16 < 4; ++k16) {
        const int row = R0 + mb * 32 + (lane & 31);
        const int q = rc + 16 * k16 + 8 * (lane >> 5);
        m[mb][k16] = (row < rows && q < capj)
                         ? *reinterpret_cast<const uint4*>(mid + (int64_t)row * L.rank_cap + rho + q)
                         : make_uint4(0, 0, 0, 0);
      }
  };

  // the wave's rows R0 + 32 mb + (lane & 31), read as one index into the LDS array (keeps the array known)
  auto load_a = [&](const uint16_t* xs, int k16, uint4 (&a)[kDMB]) __attribute__((always_inline)) {
    const int c = 2 * k16 + (lane >> 5);
    const uint4* xv = reinterpret_cast<const uint4*>(xs);
#pragma unroll
    for (int mb = 0; mb < kDMB; ++mb) a[mb] = xv[swz(R0 + mb * 32 + (lane & 31), c) >> 3];
  };
  // the wave's weight operand for 16 inputs k16: chunk (2 k16 + (lane >> 5)) * 64 + 32 cg + (lane & 31)
  // (an index the compiler cannot split, so each read's address is one offset from the buffer's start: the compiler
  // then knows which LDS array the read touches and does not wait for the x loads in flight into the x buffers)
  int wl = (lane >> 5) * kDCols + cg * 32 + (lane & 31);
  asm("" : "+v"(wl));
  auto load_w = [&](const uint4* wb, int k16) __attribute__((always_inline)) {
    return wb[wl + 2 * k16 * kDCols];
  };
  // operands of the 16-input slices k16 = h, h + 1 of a step (h = 0: the first half, h = 2: the second)
  auto read_half = [&](const uint16_t* xs, const uint4* wb, int h, uint4 (&a)[2][kDMB], uint4 (&b)[2])
      __attribute__((always_inline)) {
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      load_a(xs, h + u, a[u]);
      b[u] = load_w(wb, h + u);
    }
  };
  auto mfma_k16 = [&](const uint4 (&a)[kDMB], const uint4& b) __attribute__((always_inline)) {
#pragma unroll
    for (int mb = 0; mb < kDMB; ++mb) acc[mb] = mfma32(b, a[mb], acc[mb]);
  };

  // LoRA bookkeeping issued before the K loop so its loads land during it: each lane's row of block mb and
  // that row's segment (-1 past the pass), and the first factors of the wave's rows for the first matrix of its
  // columns (ranks 0..63); the segments' adapters and live ranks follow once the segment range is known.
  const int cw0 = GATED ? (cg ? inter : 0) + nt * 32 : n0 + cg * 32;  // the wave's first column
  const int r_end = min(R0 + 32 * kDMB, T);
  const bool lora = !RANGES && L.n_mats > 0 && mid != nullptr && cw0 < n_out && R0 < r_end;
  const int jlo = lora ? matrix_of(L, cw0) : 0;
  int rseg[kDMB];
  uint4 m0[kDMB][4];
  if (lora) {
#pragma unroll
    for (int mb = 0; mb < kDMB; ++mb) {
      const int row = R0 + mb * 32 + (lane & 31);
      rseg[mb] = row < r_end ? r.seg_of[row] : -1;
    }
    load_mid(m0, jlo, 0);
  }

  // Step i reads x buffer i % 4 (its rows loaded at the start of step i - 3) and dequantised weight buffer i % 3
  // (written late in step i - 2, after that step's barrier, from the words loaded at the start of step i - 3 into
  // register stage i % 3): a step of this narrow tile is short (8 MFMAs per wave), so the loads run three steps
  // ahead. Every load is unconditional (past the last step it re-reads the last one), so the number of loads in flight
  // at each wait is the same on every path; a step's words are issued before its x rows (loads complete in order).
  const int nk = w.k / kTK / ksplit;  // this block's K steps, from step ks * nk
  const int kbase = ks * nk * kTK;
  WStage s0, s1, s2;
  fetch_w(s0, kbase);
  dma_x(d_x0, kbase);
  fetch_w(s1, kbase + min(1, nk - 1) * kTK);
  dma_x(d_x1, kbase + min(1, nk - 1) * kTK);
  fetch_w(s2, kbase + min(2, nk - 1) * kTK);
  dma_x(d_x2, kbase + min(2, nk - 1) * kTK);
  // per block, the segments it crosses; the wave's segments (at most 64: one per row), one per lane: its adapter
  int blo[kDMB], bhi[kDMB], s_lo = 0, s_hi = -1, la = 0, llive0 = 0;
  if (lora) {
#pragma unroll
    for (int mb = 0; mb < kDMB; ++mb) {
      const int last = r_end - 1 - (R0 + mb * 32);  // the block's last row in the pass, relative to its first
      blo[mb] = last >= 0 ? __builtin_amdgcn_readfirstlane(rseg[mb]) : INT_MAX;
      bhi[mb] = last >= 0 ? __builtin_amdgcn_readlane(rseg[mb], min(last, 31)) : -1;
    }
    s_lo = blo[0];
    s_hi = bhi[kDMB - 1] >= 0 ? bhi[kDMB - 1] : bhi[0];
    la = s_lo + lane <= s_hi ? r.seg_adapter[s_lo + lane] : 0;
  }
  // landed: step 0's words and x rows and step 1's words (step 1's x rows and step 2's loads may be in flight)
  MLORA_WAIT_VM(kDXLoads + kDWLoads + kDXLoads);
  dequant_to(d_w0, s0);
  dequant_to(d_w1, s1);
  step_sync();
  uint4 a01[2][kDMB], b01[2];  // the first half of the current step's operands, read after the previous barrier
  read_half(d_x0, d_w0, 0, a01, b01);
  // One barrier per step, in its middle: the second half of step i's operands is read while the first half's MFMAs
  // run, and the first half of step i + 1's after the barrier, while the second half's MFMAs run. Before the barrier
  // the wave issues step i + 3's loads (words before x rows: loads complete in order) and waits only for step i + 1's
  // x rows; the barrier makes them visible, with step i + 1's weights (written in step i - 1). Past the barrier,
  // beside the second half's MFMAs, the wave dequantises step i + 2's words into the weight buffer step i - 1 read, so
  // the conversion is off the path from one barrier to the next.
  auto run = [&](auto slot, int i) __attribute__((always_inline)) {
    constexpr int B = decltype(slot)::value;  // i % 12
    constexpr int X = B % 4, W = B % 3;
    const uint16_t* xs = X == 0 ? d_x0 : X == 1 ? d_x1 : X == 2 ? d_x2 : d_x3;
    const uint16_t* xn = X == 0 ? d_x1 : X == 1 ? d_x2 : X == 2 ? d_x3 : d_x0;  // buffer (i + 1) % 4
    uint16_t* xf = X == 0 ? d_x3 : X == 1 ? d_x0 : X == 2 ? d_x1 : d_x2;        // buffer (i + 3) % 4
    WStage& wf = W == 0 ? s0 : W == 1 ? s1 : s2;       // step i + 3's words (fetched now into stage i % 3)
    WStage& wdq = W == 0 ? s2 : W == 1 ? s0 : s1;      // step i + 2's words (dequantised now)
    const uint4* wcur = W == 0 ? d_w0 : W == 1 ? d_w1 : d_w2;
    const uint4* wnext = W == 0 ? d_w1 : W == 1 ? d_w2 : d_w0;  // buffer (i + 1) % 3
    uint4* wfar = W == 0 ? d_w2 : W == 1 ? d_w0 : d_w1;         // buffer (i + 2) % 3
    uint4 a23[2][kDMB], b23[2];
    read_half(xs, wcur, 2, a23, b23);
    mfma_k16(a01[0], b01[0]);
    fetch_w(wf, kbase + min(i + 3, nk - 1) * kTK);
    __builtin_amdgcn_sched_barrier(0);
    mfma_k16(a01[1], b01[1]);
    dma_x(xf, kbase + min(i + 3, nk - 1) * kTK);
    __builtin_amdgcn_sched_barrier(0);
    // landed: step i + 1's x rows (step i + 2's and i + 3's loads in flight)
    MLORA_WAIT_VM(kDWLoads + kDXLoads + kDWLoads + kDXLoads);
    __builtin_amdgcn_sched_barrier(0);
    step_sync();
    read_half(xn, wnext, 0, a01, b01);  // past the last step: re-reads of valid buffers, unused
    __builtin_amdgcn_sched_barrier(0);
    mfma_k16(a23[0], b23[0]);
    mfma_k16(a23[1], b23[1]);
    // landed: step i + 2's words (its x rows and step i + 3's loads in flight)
    MLORA_WAIT_VM(kDXLoads + kDWLoads + kDXLoads);
    dequant_to(wfar, wdq);
    // after the first step, the segments' adapters have landed: their live ranks land during the next steps
    if constexpr (B == 0 && !RANGES)
      if (i == 0 && lora) llive0 = la == 0 ? 0 : live_rank(L, la, jlo);
  };
  for (int it = 0; it < nk; it += 12) steps_from<0>(run, it, nk);
  MLORA_WAIT_VM(0);
  // (the LoRA term stages sB in the ring's last two buffers: every wave's reads of the ring and x loads into it are
  // done first)
  if (!RANGES && L.n_mats > 0 && mid != nullptr) lds_sync();

  if constexpr (RANGES) {
    // this range's float32 tile, in the accumulators' order (non-temporal stores: read once, by the expand launch,
    // whose loads are non-temporal too; with plain stores and loads both launches took longer)
#pragma unroll
    for (int mb = 0; mb < kDMB; ++mb)
#pragma unroll
      for (int g = 0; g < 4; ++g)
        __builtin_nontemporal_store(
            (f32x4_t){acc[mb][4 * g], acc[mb][4 * g + 1], acc[mb][4 * g + 2], acc[mb][4 * g + 3]},
            reinterpret_cast<f32x4_t*>(&part[part_index(ks, n_tiles, nt, wave, mb, g, lane)]));
    return;
  }

  // LoRA second factor: the segments s_lo..s_hi crossing the wave's rows
  if (lora) {
    const int cc = cw0 + (lane & 31);
    const int jhi = matrix_of(L, min(cw0 + 31, n_out - 1));
    for (int j = jlo; j <= jhi; ++j) {
      const int oj = col_offset(L, j), cj = L.cols[j], capj = L.cap[j];
      const bool cin = cc >= oj && cc < oj + cj && cc < n_out;
      const bool allin = cw0 >= oj && cw0 + 32 <= oj + cj && cw0 + 32 <= n_out;  // every lane's column in matrix j
      const int llive = j == jlo ? llive0 : (la == 0 ? 0 : live_rank(L, la, j));
      for (int rc = 0; rc < capj; rc += kDRankChunk) {
        uint4 m[kDMB][4];
        if (j == jlo && rc == 0) {
#pragma unroll
          for (int mb = 0; mb < kDMB; ++mb)
#pragma unroll
            for (int k16 = 0; k16 < 4; ++k16) m[mb][k16] = m0[mb][k16];
        } else {
          load_mid(m, j, rc);
        }
        // Segment s's sB rows into an LDS slot of the wave's own (4 KB: its 32 columns x ranks rc .. rc + 63, rows
        // of 128 bytes swizzled like x), by loads that write LDS directly, one segment ahead of the segment's
        // products: instruction i fills rows 8 i + (lane >> 3) (row = the wave's column, clamped into matrix j;
        // chunks past the adapter's row re-read its last 8 ranks, masked when used), so each instruction reads 8
        // whole rows. The wave's first 64 segments are held one per lane; empty segments (requests of no tokens) can
        // put more than 64 segment indices across its 64 rows, and those past the 64th are read from memory (i is
        // uniform).
        auto load_b = [&](int s, uint16_t* slot, int& rk) __attribute__((always_inline)) {
          const int sc = min(s, s_hi), i = sc - s_lo;
          int a, live;
          if (i < kWave) {
            a = __builtin_amdgcn_readlane(la, i);
            live = __builtin_amdgcn_readlane(llive, i);
          } else {
            a = r.seg_adapter[sc];
            live = a == 0 ? 0 : live_rank(L, a, j);
          }
          rk = s <= s_hi ? min(live - rc, kDRankChunk) : 0;
          const int sbs = sb_stride(live, capj);  // at least 8: capj > rc >= 0
          MLORA_WAIT_LGKM0();                     // the wave's reads of the slot are done
          const __amdgpu_buffer_rsrc_t bres = __builtin_amdgcn_make_buffer_rsrc(
              (void*)(L.pool + (int64_t)a * L.pool_stride + L.off_b[j]), (short)0, cj * sbs * 2, 0x00020000);
#pragma unroll
          for (int i4 = 0; i4 < 4; ++i4) {
            const int row = 8 * i4 + (lane >> 3);
            const int col = cw0 - oj + row;
            const int ccr = col >= 0 && col < cj ? col : 0;
            const uint32_t off = (uint32_t)((ccr * sbs + min(rc + 8 * swz_slot(row, lane & 7), sbs - 8)) * 2);
            __builtin_amdgcn_raw_ptr_buffer_load_lds(bres, (lds_void*)(slot + i4 * 8 * kTK), 16, off, 0, 0, kReadOnce);
          }
        };
        {
          uint16_t* const slot0 = d_x2 + wave * 32 * kTK;
          uint16_t* const slot1 = d_x3 + wave * 32 * kTK;
          // the slot's operands (lane l: column l & 31, ranks 16 k16 + 8 (l >> 5) .. +7 of the chunk) once its loads
          // have landed (the next segment's 4 may be in flight), then the segment's products
          auto apply = [&](int s, const uint16_t* slot, int rk) __attribute__((always_inline)) {
            MLORA_WAIT_VM(4);
            uint4 bv[4];
            const uint4* sv = reinterpret_cast<const uint4*>(slot);
#pragma unroll
            for (int k16 = 0; k16 < 4; ++k16) bv[k16] = sv[swz(lane & 31, 2 * k16 + (lane >> 5)) >> 3];
            if (rk <= 0) return;
            uint32_t rmask[kDMB];
#pragma unroll
            for (int mb = 0; mb < kDMB; ++mb) rmask[mb] = rseg[mb] == s ? 0xFFFFFFFFu : 0u;
#pragma unroll
            for (int k16 = 0; k16 < 4; ++k16) {
              if (16 * k16 >= rk) break;
              uint4 bm = bv[k16];
              if (16 * k16 + 16 > rk) bm = keep_first(bm, rk - (16 * k16 + 8 * (lane >> 5)));
              if (!allin) bm = cin ? bm : make_uint4(0, 0, 0, 0);
#pragma unroll
              for (int mb = 0; mb < kDMB; ++mb) {
                if (s < blo[mb] || s > bhi[mb]) continue;
                const uint4 am = make_uint4(m[mb][k16].x & rmask[mb], m[mb][k16].y & rmask[mb],
                                            m[mb][k16].z & rmask[mb], m[mb][k16].w & rmask[mb]);
                acc[mb] = mfma32(bm, am, acc[mb]);
              }
            }
          };
          int k0, k1;
          load_b(s_lo, slot0, k0);
          // Each row's first factors past its own segment's live rank are set to zero once, while the first segment's
          // sB loads are in flight (the segment's live rank from its lane of llive, or from memory past the wave's
          // first 64 segments; rows past the pass have none): a segment's term then needs only a row mask on the first
          // factors, and the sB chunk crossing the live rank (rk not a multiple of 16) keeps only its live ranks, so
          // the sB row's padding never enters the sum.
#pragma unroll
          for (int mb = 0; mb < kDMB; ++mb) {
            const int sq = rseg[mb] - s_lo;
            int rrow = __builtin_amdgcn_ds_bpermute((sq & 63) << 2, llive);
            if (rseg[mb] >= 0 && sq >= kWave) {
              const int a = r.seg_adapter[rseg[mb]];
              rrow = a == 0 ? 0 : live_rank(L, a, j);
            }
            if (rseg[mb] < 0) rrow = 0;
#pragma unroll
            for (int k16 = 0; k16 < 4; ++k16)
              m[mb][k16] = keep_first(m[mb][k16], rrow - rc - (16 * k16 + 8 * (lane >> 5)));
          }
          // (no exit between the halves: past s_hi the loads re-read its last segment and rk is 0)
          for (int s = s_lo; s <= s_hi; s += 2) {
            load_b(s + 1, slot1, k1);
            apply(s, slot0, k0);
            load_b(s + 2, slot0, k0);
            apply(s + 1, slot1, k1);
          }
          MLORA_WAIT_VM(0);  // the last slot loads have landed before the slots are staged again or reused
        }
      }
    }
  }

  if constexpr (GATED) {
    // gated, one range: the up waves leave their rounded outputs in LDS (the x ring is idle after the K loop); each
    // gate wave pairs them with its own, lane for lane, and writes silu(gate) * up to output columns 32 nt .. +31
    uint2* ex = reinterpret_cast<uint2*>(d_x0);
    lds_sync();  // every wave is done reading the x ring
    if (cg == 1) {
#pragma unroll
      for (int mb = 0; mb < kDMB; ++mb)
#pragma unroll
        for (int g = 0; g < 4; ++g)
          ex[((rg * kDMB + mb) * 4 + g) * 64 + lane] = make_uint2(pack_bf16x2(acc[mb][4 * g], acc[mb][4 * g + 1]),
                                                                  pack_bf16x2(acc[mb][4 * g + 2], acc[mb][4 * g + 3]));
    }
    lds_sync();
    if (cg == 0) {
#pragma unroll
      for (int mb = 0; mb < kDMB; ++mb) {
        const int row = R0 + mb * 32 + (lane & 31);
        if (row >= T) continue;
        const int64_t orig = d_orig[row];
        const int64_t lq = d_last[row];
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const uint2 u = ex[((rg * kDMB + mb) * 4 + g) * 64 + lane];
          const uint2 v = silu_mul4(make_uint2(pack_bf16x2(acc[mb][4 * g], acc[mb][4 * g + 1]),
                                               pack_bf16x2(acc[mb][4 * g + 2], acc[mb][4 * g + 3])), u);
          const uint32_t lo = v.x, hi = v.y;
          const int col = nt * 32 + g * 8 + (lane >> 5) * 4;
          if (vec & kStoreVec) {
            *reinterpret_cast<uint2*>(y + orig * y_stride + col) = make_uint2(lo, hi);
            if (lq >= 0) *reinterpret_cast<uint2*>(last_out + lq * inter + col) = make_uint2(lo, hi);
          } else {
            const uint16_t h[4] = {(uint16_t)lo, (uint16_t)(lo >> 16), (uint16_t)hi, (uint16_t)(hi >> 16)};
            for (int e = 0; e < 4; ++e) {
              y[orig * y_stride + col + e] = h[e];
              if (lq >= 0) last_out[lq * inter + col + e] = h[e];
            }
          }
        }
      }
    }
    return;
  }
  // one range: round once and write four columns per lane and group (rows in their original order)
#pragma unroll
  for (int mb = 0; mb < kDMB; ++mb) {
    const int row = R0 + mb * 32 + (lane & 31);
    if (row >= T) continue;
    const int64_t orig = d_orig[row];
    const int64_t lq = d_last[row];
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const int col = cw0 + g * 8 + (lane >> 5) * 4;
      if (col >= n_out) continue;
      store4(y + orig * y_stride + col, lq >= 0 ? last_out + lq * n_out + col : nullptr,
             pack_bf16x2(acc[mb][4 * g], acc[mb][4 * g + 1]), pack_bf16x2(acc[mb][4 * g + 2], acc[mb][4 * g + 3]),
             n_out - col, vec);
    }
  }
}

// The expand launch: block b is (row group b % rgs, column tile b / rgs), rgs = the row groups holding tokens. Wave
// (cg, sg) covers the base launch's wave (row group, cg), its 64 rows x 32 columns, for the segments s_lo + sg,
// s_lo + sg + 4, ... crossing those rows, so a wave's few segments' sB loads are in flight at once. A row gets a LoRA
// term from its own segment only (the others' first factors are masked to zero), so the four groups' sums are exact
// zeros but for one: group 0 starts from the ranges' sum, groups 1-3 from zero, and they are added in group order
// through LDS. GATED: silu(gate) * up to inter columns.
template <bool GATED>
__global__ __launch_bounds__(kEThreads) void dec_expand_kernel(mlora_lora_t L, mlora_route_t r,
                                                               const uint16_t* __restrict__ mid,
                                                               const float4* __restrict__ part, int32_t ksplit,
                                                               int32_t n_tiles, int32_t rgs,
                                                               uint16_t* __restrict__ y, int64_t y_stride,
                                                               uint16_t* __restrict__ last_out, int32_t n_out,
                                                               int32_t vec, int32_t inter) {
  __shared__ float e_red[(kESG - 1) * kDCG * kDMB * 16 * 64];  // segment groups 1..3: their sums
  __shared__ uint2 ex[kDCG * kDMB * 4 * 64];                     // gated: the gate and up waves' rounded outputs
  const int tid = threadIdx.x, lane = tid & 63;
  const int ew = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int cg = ew % kDCG, sg = ew / kDCG;
  const int rg = blockIdx.x % rgs, nt = blockIdx.x / rgs;
  const int wave = rg * kDCG + cg;  // the base launch's wave of these rows and columns
  const int T = (int)r.tokens;
  const int R0 = rg * 32 * kDMB;
  const int r_end = min(R0 + 32 * kDMB, T);  // R0 < T: rgs row groups hold tokens
  const int cw0 = GATED ? (cg ? inter : 0) + nt * 32 : nt * kDCols + cg * 32;  // the wave's first column
  const bool lora = L.n_mats > 0 && cw0 < n_out;

  // first factors of the wave's rows R0 + 32 mb + (lane & 31), ranks rc + 16 k16 + 8 (lane >> 5) .. +7 of matrix j
  // (zero past the pass's rows and past cap_j)
  auto load_mid = [&](uint4 (&m)[kDMB][4], int j, int rc) __attribute__((always_inline)) {
    const int capj = L.cap[j], rho = rank_offset(L, j);
#pragma unroll
    for (int mb = 0; mb < kDMB; ++mb)
#pragma unroll
      for (int k16 = 0; k16 < 4; ++k16) {
        const int row = R0 + mb * 32 + (lane & 31);
        const int q = rc + 16 * k16 + 8 * (lane >> 5);
        m[mb][k16] = (row < r_end && q < capj)
                         ? *reinterpret_cast<const uint4*>(mid + (int64_t)row * L.rank_cap + rho + q)
                         : make_uint4(0, 0, 0, 0);
      }
  };

  // Everything that depends on no other load is issued first, in one round: each lane's row of block mb and that
  // row's segment (-1 past the pass), the first factors of the wave's rows for the first matrix of its columns
  // (ranks 0..63), the rows' token order for the output (group 0), the ranges' tiles (group 0). Then the two
  // dependent rounds of bookkeeping: per block, the segments it crosses, and the wave's segments (at most 64: one per
  // row), one per lane: its adapter; then the adapters' live ranks.
  const int jlo = lora ? matrix_of(L, cw0) : 0;
  int rseg[kDMB], blo[kDMB], bhi[kDMB], s_lo = 0, s_hi = -1, la = 0, llive0 = 0;
  uint4 m0[kDMB][4];
  if (lora) {
#pragma unroll
    for (int mb = 0; mb < kDMB; ++mb) {
      const int row = R0 + mb * 32 + (lane & 31);
      rseg[mb] = row < r_end ? r.seg_of[row] : -1;
    }
    load_mid(m0, jlo, 0);
  }
  int64_t orig[kDMB], lq[kDMB];
#pragma unroll
  for (int mb = 0; mb < kDMB; ++mb) {
    const int row = R0 + mb * 32 + (lane & 31);
    orig[mb] = sg == 0 && row < T ? r.tok_perm[row] : 0;
    lq[mb] = sg == 0 && row < T && last_out != nullptr ? r.last_of[row] : -1;
  }

  // (the segments' adapters are asked for before the ranges' tiles are added, so their loads run beside that sum)
  if (lora) {
#pragma unroll
    for (int mb = 0; mb < kDMB; ++mb) {
      const int last = r_end - 1 - (R0 + mb * 32);  // the block's last row in the pass, relative to its first
      blo[mb] = last >= 0 ? __builtin_amdgcn_readfirstlane(rseg[mb]) : INT_MAX;
      bhi[mb] = last >= 0 ? __builtin_amdgcn_readlane(rseg[mb], min(last, 31)) : -1;
    }
    s_lo = blo[0];
    s_hi = bhi[kDMB - 1] >= 0 ? bhi[kDMB - 1] : bhi[0];
    la = s_lo + lane <= s_hi ? r.seg_adapter[s_lo + lane] : 0;
    llive0 = la == 0 ? 0 : live_rank(L, la, jlo);
  }

  // segment group 0: the ranges' tiles added in order, four ranges' loads in flight at a time
  f32x16_t acc[kDMB];
#pragma unroll
  for (int mb = 0; mb < kDMB; ++mb) acc[mb] = f32x16_t{};
  for (int k0 = 0; k0 < (sg == 0 ? ksplit : 0); k0 += 4) {
    float4 u[4][kDMB * 4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
      if (k0 + i < ksplit)
#pragma unroll
        for (int e = 0; e < kDMB * 4; ++e) {
          const f32x4_t v = __builtin_nontemporal_load(
              reinterpret_cast<const f32x4_t*>(&part[part_index(k0 + i, n_tiles, nt, wave, e / 4, e % 4, lane)]));
          u[i][e] = make_float4(v.x, v.y, v.z, v.w);
        }
#pragma unroll
    for (int i = 0; i < 4; ++i)
      if (k0 + i < ksplit)
#pragma unroll
        for (int e = 0; e < kDMB * 4; ++e) {
          const int mb = e / 4, g = e % 4;
          if (k0 + i == 0) {
            acc[mb][4 * g] = u[i][e].x;
            acc[mb][4 * g + 1] = u[i][e].y;
            acc[mb][4 * g + 2] = u[i][e].z;
            acc[mb][4 * g + 3] = u[i][e].w;
          } else {
            acc[mb][4 * g] += u[i][e].x;
            acc[mb][4 * g + 1] += u[i][e].y;
            acc[mb][4 * g + 2] += u[i][e].z;
            acc[mb][4 * g + 3] += u[i][e].w;
          }
        }
  }

  // LoRA second factor: the wave's share of the segments s_lo..s_hi crossing its rows
  if (lora) {
    const int cc = cw0 + (lane & 31);
    const int jhi = matrix_of(L, min(cw0 + 31, n_out - 1));
    for (int j = jlo; j <= jhi; ++j) {
      const int oj = col_offset(L, j), cj = L.cols[j], capj = L.cap[j];
      const bool cin = cc >= oj && cc < oj + cj && cc < n_out;
      const bool allin = cw0 >= oj && cw0 + 32 <= oj + cj && cw0 + 32 <= n_out;  // every lane's column in matrix j
      const int llive = j == jlo ? llive0 : (la == 0 ? 0 : live_rank(L, la, j));
      for (int rc = 0; rc < capj; rc += kDRankChunk) {
        uint4 m[kDMB][4];
        if (j == jlo && rc == 0) {
#pragma unroll
          for (int mb = 0; mb < kDMB; ++mb)
#pragma unroll
            for (int k16 = 0; k16 < 4; ++k16) m[mb][k16] = m0[mb][k16];
        } else {
          load_mid(m, j, rc);
        }
        // Segment s's sB rows into an LDS slot of the wave's own (its 32 columns x ranks rc .. rc + 63, rows of 128
        // bytes swizzled like x) by loads that write LDS directly, each instruction 8 whole rows (row = the wave's
        // column, clamped into matrix j; chunks past the adapter's row re-read its last 8 ranks, masked when used),
        // one of the wave's segments ahead of its products. The wave's first 64 segments are held one per lane; empty
        // segments (requests of no tokens) can put more than 64 segment indices across its 64 rows, and those past
        // the 64th are read from memory (i is uniform).
        auto load_b = [&](int s, uint16_t* slot, int& rk) __attribute__((always_inline)) {
          const int sc = min(s, s_hi), i = sc - s_lo;
          int a, live;
          if (i < kWave) {
            a = __builtin_amdgcn_readlane(la, i);
            live = __builtin_amdgcn_readlane(llive, i);
          } else {
            a = r.seg_adapter[sc];
            live = a == 0 ? 0 : live_rank(L, a, j);
          }
          rk = s <= s_hi ? min(live - rc, kDRankChunk) : 0;
          const int sbs = sb_stride(live, capj);  // at least 8: capj > rc >= 0
          MLORA_WAIT_LGKM0();                     // the wave's reads of the slot are done
          const uint16_t* blk = L.pool + (int64_t)a * L.pool_stride + L.off_b[j];
          // (through a buffer resource; the gated form, whose scalar registers are fewer to spare, by 64-bit
          // addresses: with the resource it reserved a scratch frame)
          const __amdgpu_buffer_rsrc_t bres =
              __builtin_amdgcn_make_buffer_rsrc((void*)blk, (short)0, GATED ? 0 : cj * sbs * 2, 0x00020000);
#pragma unroll
          for (int i4 = 0; i4 < 4; ++i4) {
            const int row = 8 * i4 + (lane >> 3);
            const int col = cw0 - oj + row;
            const int ccr = col >= 0 && col < cj ? col : 0;
            const int q = ccr * sbs + min(rc + 8 * swz_slot(row, lane & 7), sbs - 8);
            if constexpr (GATED)
              __builtin_amdgcn_global_load_lds((const void*)(blk + q), (lds_void*)(slot + i4 * 8 * kTK), 16, 0, kReadOnce);
            else
              __builtin_amdgcn_raw_ptr_buffer_load_lds(bres, (lds_void*)(slot + i4 * 8 * kTK), 16, (uint32_t)q * 2, 0,
                                                       0, kReadOnce);
          }
        };
        uint16_t* const slot0 = d_x2 + ew * 32 * kTK;  // (the base launch's x buffers: 4 KB a wave in each)
        uint16_t* const slot1 = d_x3 + ew * 32 * kTK;
        // the slot's operands (lane l: column l & 31, ranks 16 k16 + 8 (l >> 5) .. +7 of the chunk) once its loads
        // have landed (the next segment's 4 may be in flight), then the segment's products
        auto apply = [&](int s, const uint16_t* slot, int rk) __attribute__((always_inline)) {
          MLORA_WAIT_VM(4);
          uint4 bv[4];
          const uint4* sv = reinterpret_cast<const uint4*>(slot);
#pragma unroll
          for (int k16 = 0; k16 < 4; ++k16) bv[k16] = sv[swz(lane & 31, 2 * k16 + (lane >> 5)) >> 3];
          if (rk <= 0) return;
          uint32_t rmask[kDMB];
#pragma unroll
          for (int mb = 0; mb < kDMB; ++mb) rmask[mb] = rseg[mb] == s ? 0xFFFFFFFFu : 0u;
#pragma unroll
          for (int k16 = 0; k16 < 4; ++k16) {
            if (16 * k16 >= rk) break;
            uint4 bm = bv[k16];
            if (16 * k16 + 16 > rk) bm = keep_first(bm, rk - (16 * k16 + 8 * (lane >> 5)));
            if (!allin) bm = cin ? bm : make_uint4(0, 0, 0, 0);
#pragma unroll
            for (int mb = 0; mb < kDMB; ++mb) {
              if (s < blo[mb] || s > bhi[mb]) continue;
              const uint4 am = make_uint4(m[mb][k16].x & rmask[mb], m[mb][k16].y & rmask[mb],
                                          m[mb][k16].z & rmask[mb], m[mb][k16].w & rmask[mb]);
              acc[mb] = mfma32(bm, am, acc[mb]);
            }
          }
        };
        int k0, k1;
        load_b(s_lo + sg, slot0, k0);
        // Each row's first factors past its own segment's live rank are set to zero once, while the first segment's
        // sB loads are in flight (the segment's live rank from its lane of llive, or from memory past the wave's
        // first 64 segments; rows past the pass have none): a segment's term then needs only a row mask on the first
        // factors, and the sB chunk crossing the live rank (rk not a multiple of 16) keeps only its live ranks, so
        // the sB row's padding never enters the sum.
#pragma unroll
        for (int mb = 0; mb < kDMB; ++mb) {
          const int sq = rseg[mb] - s_lo;
          int rrow = __builtin_amdgcn_ds_bpermute((sq & 63) << 2, llive);
          if (rseg[mb] >= 0 && sq >= kWave) {
            const int a = r.seg_adapter[rseg[mb]];
            rrow = a == 0 ? 0 : live_rank(L, a, j);
          }
          if (rseg[mb] < 0) rrow = 0;
#pragma unroll
          for (int k16 = 0; k16 < 4; ++k16)
            m[mb][k16] = keep_first(m[mb][k16], rrow - rc - (16 * k16 + 8 * (lane >> 5)));
        }
        // (no exit between the halves: past s_hi the loads re-read its last segment and rk is 0)
        for (int s = s_lo + sg; s <= s_hi; s += 2 * kESG) {
          load_b(s + kESG, slot1, k1);
          apply(s, slot0, k0);
          load_b(s + 2 * kESG, slot0, k0);
          apply(s + kESG, slot1, k1);
        }
        MLORA_WAIT_VM(0);  // the last slot loads have landed before the slots are staged again
      }
    }
  }

  // segment groups 1..3 hand their sums to group 0, which adds them in order
  float* red = e_red + (size_t)((sg - 1) * kDCG + cg) * (kDMB * 16 * 64);
  if (sg > 0) {
#pragma unroll
    for (int mb = 0; mb < kDMB; ++mb)
#pragma unroll
      for (int i = 0; i < 16; ++i) red[(mb * 16 + i) * 64 + lane] = acc[mb][i];
  }
  lds_sync();
  if (sg == 0) {
    for (int g = 1; g < kESG; ++g) {
      const float* rg_sum = e_red + (size_t)((g - 1) * kDCG + cg) * (kDMB * 16 * 64);
#pragma unroll
      for (int mb = 0; mb < kDMB; ++mb)
#pragma unroll
        for (int i = 0; i < 16; ++i) acc[mb][i] += rg_sum[(mb * 16 + i) * 64 + lane];
    }
  }
  if constexpr (GATED) {
    // the gate and up waves leave their rounded outputs in LDS; then wave cg pairs gate and up of row block cg, lane
    // for lane, and writes silu(gate) * up to output columns 32 nt .. +31
    static_assert(kDMB == kDCG, "one row block per column group's wave");
    if (sg == 0) {
#pragma unroll
      for (int mb = 0; mb < kDMB; ++mb)
#pragma unroll
        for (int g = 0; g < 4; ++g)
          ex[((cg * kDMB + mb) * 4 + g) * 64 + lane] = make_uint2(pack_bf16x2(acc[mb][4 * g], acc[mb][4 * g + 1]),
                                                                  pack_bf16x2(acc[mb][4 * g + 2], acc[mb][4 * g + 3]));
    }
    lds_sync();
    const int mb = cg, row = R0 + mb * 32 + (lane & 31);
    if (sg != 0 || row >= T) return;
    const int64_t o = cg == 0 ? orig[0] : orig[1], q = cg == 0 ? lq[0] : lq[1];
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const uint2 v = silu_mul4(ex[(mb * 4 + g) * 64 + lane], ex[((kDMB + mb) * 4 + g) * 64 + lane]);
      const int col = nt * 32 + g * 8 + (lane >> 5) * 4;
      store4(y + o * y_stride + col, q >= 0 ? last_out + q * inter + col : nullptr, v.x, v.y, 4, vec & kStoreVec);
    }
    return;
  }
  // round once and write four columns per lane and group (rows in their original order)
  if (sg != 0) return;
#pragma unroll
  for (int mb = 0; mb < kDMB; ++mb) {
    const int row = R0 + mb * 32 + (lane & 31);
    if (row >= T) continue;
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const int col = cw0 + g * 8 + (lane >> 5) * 4;
      if (col >= n_out) continue;
      store4(y + orig[mb] * y_stride + col, lq[mb] >= 0 ? last_out + lq[mb] * n_out + col : nullptr,
             pack_bf16x2(acc[mb][4 * g], acc[mb][4 * g + 1]), pack_bf16x2(acc[mb][4 * g + 2], acc[mb][4 * g + 3]),
             n_out - col, vec);
    }
  }
}

}  // namespace

size_t dec_partials_bytes(const mlora_int4_t& w, int32_t ksplit) {
  if (ksplit <= 1) return 0;
  return (size_t)ksplit * (size_t)(w.columns / kDCols) * kDRows * kDCols * 4;
}

int launch_dec(const mlora_int4_t& w, const mlora_lora_t& L, const mlora_route_t& r, const uint16_t* x,
               int64_t x_stride, uint16_t* y, int64_t y_stride, uint16_t* last_out, int32_t n_out, uint16_t* mid,
               bool shrink, float* part, int32_t ksplit, hipStream_t stream, int32_t inter, bool residual) {
  if (r.tokens == 0 || n_out == 0) return MLORA_OK;
  if (ksplit < 1 || ksplit > kDMaxRanges) return MLORA_EINVAL;
  if (r.tokens > kDRows || w.columns % kDCols || (w.k / kTK) % ksplit || (residual && inter > 0)) return MLORA_EINVAL;
  if (inter > 0 && (inter % 32 || n_out != 2 * inter)) return MLORA_EINVAL;
  if (ksplit > 1 && part == nullptr) return MLORA_EWORKSPACE;
  const int n_tiles = inter > 0 ? inter / 32 : w.columns / kDCols;
  const int out_cols = inter > 0 ? inter : n_out;  // columns of y and last_out
  // 8-byte stores of four columns need 8-byte aligned output rows
  const int32_t vec = (reinterpret_cast<uintptr_t>(y) % 8 == 0 && y_stride % 4 == 0 &&
                       (last_out == nullptr || (reinterpret_cast<uintptr_t>(last_out) % 8 == 0 && out_cols % 4 == 0))
                           ? kStoreVec
                           : 0) |
                      (residual ? kStoreResidual : 0);
  if (ksplit == 1) {
    // the first factors, then the tiles with the LoRA term
    if (shrink) {
      const int rc = launch_shrink(L, r, x, x_stride, w.k, mid, false, stream);
      if (rc) return rc;
    }
    hipLaunchKernelGGL((inter > 0 ? dec_kernel<true, false> : dec_kernel<false, false>), dim3((unsigned)n_tiles),
                       dim3(kDThreads), 0, stream, w, L, r, x, x_stride, y, y_stride, last_out, n_out, mid, n_tiles,
                       vec, nullptr, 1, inter, 0);
    return hipGetLastError() == hipSuccess ? MLORA_OK : MLORA_ELAUNCH;
  }
  // first-factor blocks: every (segment, 32-rank block) pair of the route's capacity
  int max_blocks = 0;
  for (int j = 0; j < L.n_mats; ++j) max_blocks += (L.cap[j] + 31) / 32;
  const int64_t shrink_blocks = shrink ? (int64_t)r.max_segs * max_blocks : 0;
  if (shrink_blocks + (int64_t)n_tiles * ksplit > INT_MAX) return MLORA_EOVERFLOW;
  float4* p4 = reinterpret_cast<float4*>(part);
  hipLaunchKernelGGL((inter > 0 ? dec_kernel<true, true> : dec_kernel<false, true>),
                     dim3((unsigned)(shrink_blocks + n_tiles * ksplit)), dim3(kDThreads), 0, stream, w, L, r, x,
                     x_stride, y, y_stride, last_out, n_out, mid, n_tiles, vec, p4, ksplit, inter,
                     max_blocks);
  if (hipGetLastError() != hipSuccess) return MLORA_ELAUNCH;
  const int rgs = (int)((r.tokens + 32 * kDMB - 1) / (32 * kDMB));  // row groups holding tokens
  const dim3 grid((unsigned)(n_tiles * rgs));
  if (inter > 0)
    hipLaunchKernelGGL(dec_expand_kernel<true>, grid, dim3(kEThreads), 0, stream, L, r, mid, p4, ksplit, n_tiles,
                       rgs, y, y_stride, last_out, n_out, vec, inter);
  else
    hipLaunchKernelGGL(dec_expand_kernel<false>, grid, dim3(kEThreads), 0, stream, L, r, mid, p4, ksplit, n_tiles,
                       rgs, y, y_stride, last_out, n_out, vec, inter);
  return hipGetLastError() == hipSuccess ? MLORA_OK : MLORA_ELAUNCH;
}
