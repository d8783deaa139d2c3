// Prefill-sized INT4 base product with the LoRA second factor fused (the same arithmetic as base.hip's kernels):
//   y[perm[p], c] = bf16( sum_k x[perm[p], k] W[c, k] + sum_q mid[p, rho_j + q] sB_j[a][c - o_j, q] )
// Tiles of 256 sorted tokens x 256 columns, 8 waves of 256 x 32 (each wave all of the tile's rows and its own 32
// columns), 32x32x16 bf16 MFMA, float32 accumulators; two waves per SIMD. The MFMAs take the weights as their first
// operand, so each lane's accumulators hold four consecutive output columns of one token row. A wave owning its
// columns alone dequantises each weight once per tile (8 MFMAs per dequantised word); the price is that every wave
// reads all 256 rows of x from LDS.
//
// Per K step of 64 inputs:
//  - x: the 256 gathered rows go straight from memory to LDS (buffer loads with the LDS flag, 16 bytes per lane, no
//    registers), two steps ahead, into a ring of three LDS buffers; the waves read their operands from it;
//  - weights: no LDS at all. Each lane loads the packed words that form its own operands (one 32-bit word = the 8
//    consecutive inputs of one column that a 32x32x16 operand lane holds), one step ahead, with the raw scale and
//    zero point of its columns, and dequantises them to bf16((c - z) s) in registers, the next 16 inputs' words
//    interleaved with the current MFMAs.
// With no LDS stores in the loop, nothing but the x ring is ordered by the step barrier: a bare barrier after an
// explicit wait for the x rows of the next step (a __syncthreads(), or any release fence, would also wait for the
// rows two steps ahead).
// LDS rows are 128 bytes (64 bf16) with their eight 16-byte chunks XOR-swizzled by (row >> 1) & 7 (tile_common.h's
// swz): the 16-byte operand reads of 16 consecutive rows hit all 64 banks once. The ring buffers are distinct LDS
// arrays chosen at compile time (the loop is unrolled by six). Tiles are ordered so that the column tiles of one
// row tile run on the same XCD (its x rows, the larger operand, then come from that XCD's L2).
// Epilogue: the tile's first factors (sorted rows) are staged in LDS; each adapter segment crossing the tile adds
// its sB rows (loaded straight into operands, segments ahead) times the first factors of its rows by MFMA; then the
// single rounding to bf16, staged through LDS so every output row is written in whole 512-byte pieces. Decode-shaped
// passes (few tokens per segment) alternate: odd row tiles add their LoRA term before the K loop.
#include <type_traits>

#include "tile_common.h"

namespace {

using namespace mlora;
typedef unsigned u32x4_t __attribute__((ext_vector_type(4)));  // (the non-temporal store's operand type)

constexpr int kTM = 256, kTN = 256;
constexpr int kThreads = 512;
constexpr int kRankChunk = 64;   // ranks of sB staged per epilogue pass
constexpr int kXLoads = 4;       // global_load_lds instructions per lane and step
constexpr int kWLoads = 4 + 2;   // weight loads per lane and step: 4 words, a scale, a zero point
constexpr int32_t kLoraEarly = 4;  // `vec` bit: odd row tiles add the LoRA term before the K loop

__shared__ __attribute__((aligned(16))) uint16_t g_x0[kTM * kTK];
__shared__ __attribute__((aligned(16))) uint16_t g_x1[kTM * kTK];
__shared__ __attribute__((aligned(16))) uint16_t g_x2[kTM * kTK];
__shared__ __attribute__((aligned(16))) uint16_t g_x3[kTM * kTK];  // the output tile's staging only
__shared__ int32_t g_orig[kTM];  // the tile's rows: original token index, -1 past the tokens
__shared__ int32_t g_last[kTM];  // the tile's rows: request whose last token it is, else -1

// MB: 32-row blocks of a tile (8: 256 rows; 7: 224 and 4: 128 rows, chosen by the host when they take fewer rounds
// of tiles);
// GATED: the gated epilogue (silu(gate) * up, inter columns), a template parameter so the plain kernel carries none of it;
// EARLY: the kernel may add the LoRA term before the K loop (decode-shaped passes, below). The prefill kernels carry
// no such path: with it, the compiler waits for every load in flight at the top of each round of the K loop. The
// EARLY kernels also write their output tiles with non-temporal stores (decode-pool-28l's step 32.5 -> 31.6 ms: less
// left to write back at each launch's end); a long prefill launch measured no better, or slightly worse, with them.
template <int MB, bool GATED, bool EARLY>
__global__ __launch_bounds__(kThreads) void base_mfma256_kernel(mlora_int4_t w, mlora_lora_t L, mlora_route_t r,
                                                               const uint16_t* __restrict__ x, int64_t x_stride,
                                                               uint16_t* __restrict__ y, int64_t y_stride,
                                                               uint16_t* __restrict__ last_out, int32_t n_out,
                                                               const uint16_t* __restrict__ mid, int32_t n_tiles,
                                                               int32_t vec,  // kStoreVec | kStoreResidual
                                                               float* __restrict__ part, int32_t ksplit,
                                                               int32_t base_blocks, int32_t inter) {
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform: LDS addresses of the x loads in SGPRs
  // Block b -> (K range ks, row tile mt, column tile nt), column tiles innermost: the blocks that share x rows (one
  // row tile and K range) are consecutive and so run on one XCD.
  const int b = xcd_tile(blockIdx.x, base_blocks);
  const int t = b % (base_blocks / ksplit), ks = b / (base_blocks / ksplit);
  // Decode-shaped passes (kLoraEarly) take the row tiles in pairs, column tiles interleaved (2m, 0), (2m + 1, 0),
  // (2m, 1), ...: the two tiles of a pair add their LoRA terms at different times (below), and a round of an XCD's
  // workgroups then holds as many of each, where row tiles taken whole fill a round with one kind.
  int mt, nt;
  if (vec & kLoraEarly) {
    const int m_tiles = base_blocks / ksplit / n_tiles, full = (m_tiles & ~1) * n_tiles;
    mt = t < full ? (t / (2 * n_tiles)) * 2 + (t & 1) : m_tiles - 1;
    nt = t < full ? (t % (2 * n_tiles)) >> 1 : t - full;
  } else {
    mt = t / n_tiles;
    nt = t - mt * n_tiles;
  }
  const int64_t T = r.tokens;
  constexpr int kRows = 32 * MB;  // the tile's rows (LDS buffers hold 256; rows past kRows are loaded, never used)
  const int64_t p0 = (int64_t)mt * kRows;
  const int n0 = nt * kTN;
  // The wave's first column: its 32 of the tile's 256; in a gated product (inter > 0: gate columns [0, inter), up
  // columns [inter, 2 inter)) the tile pairs gate columns 128 nt .. +127 (waves 0..3) with the same up columns
  // (waves 4..7), and writes silu(gate) * up to output columns 128 nt .. +127.
  const int wc0 = GATED ? (wave < 4 ? 0 : inter) + nt * 128 + (wave & 3) * 32 : n0 + wave * 32;

  // Loads go through buffer resources: the per-lane byte offsets below stay fixed for the whole K loop and the K
  // position is a wave-uniform scalar offset, so no 64-bit addresses are kept in registers. The resources' sizes
  // are the arrays' sizes, except for x, gathered row by row, whose resource spans the whole 32-bit range (the host
  // keeps tokens x x_stride below 2^31 elements, so every byte offset fits 32 bits).
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

  // x: instruction i of wave `wave` fills rows (8 i + wave) * 8 .. +7; lane l writes LDS chunk slot l & 7 of row
  // +(l >> 3), which holds logical chunk swz_slot(row, l & 7). Rows past the tokens read row 0 of the pass.
  if (tid < kTM) {
    const int64_t p = p0 + tid;
    const bool mine = tid < kRows && p < T;
    g_orig[tid] = mine ? r.tok_perm[p] : -1;
    g_last[tid] = (mine && last_out != nullptr) ? r.last_of[p] : -1;
  }
  uint32_t xoff[kXLoads];
#pragma unroll
  for (int i = 0; i < kXLoads; ++i) {
    const int row = (8 * i + wave) * 8 + (lane >> 3);
    const int64_t p = p0 + row;
    xoff[i] = (uint32_t)(((int64_t)r.tok_perm[p < T ? p : 0] * x_stride + (swz_slot(row, lane & 7) << 3)) * 2);
  }
  auto dma_x = [&](uint16_t* buf, int kc) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < kXLoads; ++i)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(xres, (lds_void*)(buf + (8 * i + wave) * 8 * kTK), 16, xoff[i], kc * 2,
                                               0, 0);
  };

  // weights: lane l of wave w holds column n0 + 32 w + (l & 31) and, for 16 inputs k16, the word of inputs
  // 16 k16 + 8 (l >> 5) .. +7; columns past the layout read column 0 and get zero weights (scale 0)
  const int wcol = wc0 + (lane & 31);
  const bool colok = wcol < w.columns;
  const uint32_t gcol = colok ? wcol : 0;
  const uint32_t woff = (gcol + (uint32_t)(lane >> 5) * w.columns) * 4;
  const uint32_t soff = gcol * 2;
  const uint32_t zoff = asym ? gcol : gcol * 2;
  const int wstep = w.columns * 8;  // bytes between the words of k16 and k16 + 1
  auto fetch_w = [&](WStage& st, int kc) __attribute__((always_inline)) {
    const int wbase = (kc / 8) * w.columns * 4;
#pragma unroll
    for (int k16 = 0; k16 < 4; ++k16) st.w[k16] = __builtin_amdgcn_raw_buffer_load_b32(wres, woff, wbase + k16 * wstep, 0);
    const int g = (kc >> gshift) * w.columns;
    st.sbits = __builtin_amdgcn_raw_buffer_load_b16(sres, soff, g * 2, 0);
    st.zbyte = __builtin_amdgcn_raw_buffer_load_b8(zres, zoff, asym ? g : g * 2, 0);
  };

  f32x16_t acc[MB];
#pragma unroll
  for (int mb = 0; mb < MB; ++mb) acc[mb] = f32x16_t{};

  // (indexed as 16-byte elements of the buffer: each read's address is then one index into the LDS array, which
  // keeps the compiler's knowledge of which array it reads, so it does not wait for x loads into the other buffers)
  auto load_a = [&](const uint16_t* xs, int k16, uint4 (&a)[MB]) __attribute__((always_inline)) {
    const int c = 2 * k16 + (lane >> 5);
    const uint4* xv = reinterpret_cast<const uint4*>(xs);
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) a[mb] = xv[swz(mb * 32 + (lane & 31), c) >> 3];
  };
  // One K step: A operands from the x buffer, B operands dequantised in registers from the step's words. Each A
  // operand register is reloaded right after its MFMA with the next 16 inputs' operand (it is used again eight MFMAs
  // later), and the next word's dequantisation is interleaved with the MFMAs (one MFMA, then a few VALU instructions
  // and an LDS read), so the matrix core works while the wave converts. The step's barrier sits before its last 16
  // inputs: past it, the wave reloads its A registers with the next step's first operands (buffer xn) while the last
  // MFMAs run. a holds the step's first A operands on entry.
  uint4 a[MB];
  auto step = [&](const uint16_t* xs, const WStage& ws, const uint16_t* xn, auto&& loads_w, auto&& loads_x)
      __attribute__((always_inline)) {
    const float s0v = bf16_to_f32(ws.sbits);
    const float zv = asym ? (float)ws.zbyte : 8.0f;
    const float sv = colok ? s0v : 0.0f;
    const float zs = colok ? zv * s0v : 0.0f;
    uint4 b0 = dequant_word(ws.w[0], sv, zs), b1;
#pragma unroll
    for (int k16 = 0; k16 < kTK / 16; ++k16) {
      const uint4& cb = (k16 & 1) ? b1 : b0;
      uint4& nbv = (k16 & 1) ? b0 : b1;
      if (k16 == kTK / 16 - 1) {
        __builtin_amdgcn_sched_barrier(0);
        MLORA_WAIT_VM(kWLoads + kXLoads);  // x(i + 1) has landed
        step_sync();
      }
      if (k16 + 1 < kTK / 16) nbv = dequant_word(ws.w[k16 + 1], sv, zs);
      if (k16 == 0) loads_w();
      if (k16 == 1) loads_x();
      const uint16_t* src = k16 + 1 < kTK / 16 ? xs : xn;
      const int c = 2 * ((k16 + 1) % (kTK / 16)) + (lane >> 5);
      const uint4* xv = reinterpret_cast<const uint4*>(src);
#pragma unroll
      for (int mb = 0; mb < MB; ++mb) {
        acc[mb] = mfma32(cb, a[mb], acc[mb]);
        a[mb] = xv[swz(mb * 32 + (lane & 31), c) >> 3];
      }
#pragma unroll
      for (int i = 0; i < MB; ++i) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // one MFMA
        __builtin_amdgcn_sched_group_barrier(0x002, 3, 0);  // three VALU
        __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // one LDS read
        if ((k16 == 0 && i < kWLoads) || (k16 == 1 && i < kXLoads))
          __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);  // one load
      }
      __builtin_amdgcn_sched_barrier(0);  // a reload stays eight MFMAs ahead of its use
    }
  };

  // Step i reads x buffer i % 3 (its rows loaded at the start of step i - 2) and weight set i % 2 (loaded at the
  // start of step i - 1). Every load is unconditional (past the last step it re-reads the last one into a buffer or
  // set that is never used), so the number of loads in flight at each wait is the same on every path. Each step
  // issues its weights before its x rows: loads complete in order, so waiting for the weights of step i + 1 does not
  // wait for the x rows of step i + 2. After x(i + 1) come w(i + 1) and x(i + 2).
  const int nk = w.k / kTK / ksplit;  // this block's K steps, from step ks * nk
  const int kbase = ks * nk * kTK;
  // Decode-shaped passes (kLoraEarly, set by the host for short segments) alternate the LoRA term's place by row tile:
  // odd row tiles add it before their K loop, so while some workgroups stream sB from memory others run their MFMA
  // loops. The order depends on the row tile alone, and the gated and plain forms of a group cut the same row tiles,
  // so an output's sum is formed in the same order in both. Such a tile loads its first x rows after the term, whose
  // sB slots are in their buffers.
  const bool lora = part == nullptr && L.n_mats > 0 && mid != nullptr;
  const bool early = EARLY && lora && (vec & kLoraEarly) && (mt & 1);
  WStage s0, s1;
  fetch_w(s0, kbase);
  if (!early) {
    dma_x(g_x0, kbase);
    dma_x(g_x1, kbase + min(1, nk - 1) * kTK);
  }
  // The LoRA epilogue's bookkeeping, read while the first x rows load (scalar loads, which the vector-memory waits do
  // not count): the tile's first and last adapter segments, the first two segments' adapters and their live ranks of
  // the tile's first matrix.
  const int jlo = lora ? matrix_of(L, GATED ? nt * 128 : n0) : 0;
  // (each pair packed in one 64-bit word, segment s_lo's in the low half: an array indexed by the segment would be
  // placed in scratch memory)
  int s_lo = 0, s_hi = -1;
  uint64_t a_pre = 0, live_pre = 0, live_up = 0;
  if (lora) {
    auto sload = [](const int32_t* q, int64_t i) __attribute__((always_inline)) {
      return ((const __attribute__((address_space(4))) int32_t*)(uintptr_t)q)[i];
    };
    s_lo = sload(r.seg_of, p0);
    s_hi = sload(r.seg_of, min(p0 + kRows, T) - 1);
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int a = sload(r.seg_adapter, u == 0 ? s_lo : min(s_lo + 1, s_hi));
      const int rk = a == 0 ? 0 : sload(L.ranks, (int64_t)a * L.ranks_stride + jlo);
      a_pre |= (uint64_t)(uint32_t)a << (32 * u);
      live_pre |= (uint64_t)(uint32_t)min(max(rk, 0), L.cap[jlo]) << (32 * u);
      if constexpr (GATED) {  // and of the up matrix, which waves 4..7 add
        const int ru = a == 0 ? 0 : sload(L.ranks, (int64_t)a * L.ranks_stride + 1);
        live_up |= (uint64_t)(uint32_t)min(max(ru, 0), L.cap[1]) << (32 * u);
      }
    }
  }
  auto half_of = [](uint64_t pair, int i) __attribute__((always_inline)) { return (int)(uint32_t)(pair >> (32 * i)); };
  // LoRA second factor. The tile's rows of the first factor (sorted order, 64 ranks of a matrix at a time) are staged
  // in LDS once; then for each adapter segment crossing the tile the wave stages its sB rows (its 32 columns x 64
  // ranks: 32 rows of 128 bytes) in an LDS slot of its own, one segment ahead of their products, by loads that write
  // LDS directly, each instruction reading 8 whole 128-byte rows (loaded as MFMA operands, lane = column, each
  // instruction touches 32 rows in 32-byte pieces, and a workgroup streams at about half the rate); the products are
  // added with the first factors of rows outside the segment, and ranks past the adapter's live rank, set to zero. A
  // decode-shaped tile
  // crosses ~64 segments, so their bookkeeping is read into lane tables (lane i: segment c0 + i's adapter, live rank
  // and bounds, 64 segments at a time) and taken with readlane, with no memory latency per segment; the first two
  // segments' adapters and live ranks of the first matrix were read in the prologue, so a prefill tile (one or two
  // segments) starts its sB loads at once. st0 (and st1, the gated form's second buffer) are the LDS buffers the first
  // factors are staged in: after the K loop any of the ring; before it (`early`) the two the loop writes last (g_x3 is
  // the output tile's only; g_x2 is first written by the loop's first step, after a barrier).
  // sl0, sl1: the two LDS buffers of the slots (the wave's at 32 x 64 elements from their starts).
  auto lora_term = [&](uint16_t* st0, uint16_t* st1, uint16_t* sl0, uint16_t* sl1) __attribute__((always_inline)) {
    const __amdgpu_buffer_rsrc_t mres = __builtin_amdgcn_make_buffer_rsrc(
        (void*)mid, (short)0, (int)((int64_t)T * L.rank_cap * 2), 0x00020000);  // < 2^31: checked on the host
    uint16_t* const slot0 = sl0 + wave * 32 * kTK;
    uint16_t* const slot1 = sl1 + wave * 32 * kTK;
    // A segment's sB rows into a slot: row i is column c0 + i of matrix j (rows past the matrix read its column 0 and
    // are never used), ranks rc .. rc + 63 of the adapter's row stride sbs (chunks past the row re-read its last 8:
    // past the live rank, masked when used). Instruction i fills rows 8 i + (lane >> 3); lane l writes slot l & 7 of
    // its row, which holds the row's 16-byte chunk swz_slot(row, l & 7), as in the x rows.
    auto stage_b = [&](uint16_t* slot, const uint16_t* blk, int sbs, int rc, int c0, int cj)
        __attribute__((always_inline)) {
      MLORA_WAIT_LGKM0();  // the wave's reads of the slot are done
      const __amdgpu_buffer_rsrc_t bres =
          __builtin_amdgcn_make_buffer_rsrc((void*)blk, (short)0, cj * sbs * 2, 0x00020000);  // the matrix's sB
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int row = 8 * i + (lane >> 3);
        const int col = c0 + row;
        const int ccr = col >= 0 && col < cj ? col : 0;
        const uint32_t off = (uint32_t)((ccr * sbs + min(rc + 8 * swz_slot(row, lane & 7), sbs - 8)) * 2);
        // (read once in decode-shaped passes, whose segments fit a row tile; a prefill segment's sB is re-read by
        // each of its row tiles and stays cacheable)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(bres, (lds_void*)(slot + i * 8 * kTK), 16, off, 0, 0,
                                                 EARLY ? kReadOnce : 0);
      }
    };
    // the wave's operands of a staged segment (lane l: column l & 31, ranks 16 k16 + 8 (l >> 5) .. +7 of the chunk),
    // once its slot's loads have landed (the next segment's 4 may be in flight)
    auto read_b = [&](const uint16_t* slot, uint4 (&bv)[4]) __attribute__((always_inline)) {
      MLORA_WAIT_VM(4);
      const uint4* sv = reinterpret_cast<const uint4*>(slot);
#pragma unroll
      for (int k16 = 0; k16 < 4; ++k16) bv[k16] = sv[swz(lane & 31, 2 * k16 + (lane >> 5)) >> 3];
    };
    // one pass over the segments: `stage` stages the first factors, then per chunk of 64 segments the lane tables
    // (ta, tb, te: adapter and bounds; tl: live rank of matrix j) and the segments' products, sB one ahead.
    // `ahead`: the prologue's read-ahead applies (the first chunk of matrix jlo); `rc` the rank chunk
    auto pass = [&](int j, int rc, bool ahead, auto&& stage, auto&& load_seg, auto&& apply_seg)
        __attribute__((always_inline)) {
      stage();
      __builtin_amdgcn_sched_barrier(0);  // the staging loads are issued before every load below
      for (int c0 = s_lo; c0 <= s_hi; c0 += kWave) {
        const int cend = min(c0 + kWave - 1, s_hi);  // the chunk's last segment
        const int sc = min(c0 + lane, cend);
        const int ta = r.seg_adapter[sc], tb = r.seg_start[sc], te = r.seg_start[sc + 1];
        const int tl = ta == 0 ? 0 : live_rank(L, ta, j);
        const bool pre = ahead && c0 == s_lo;
        // segment s's adapter and live rank (s clamped to the chunk: past it the loads re-read its last segment and
        // rk is 0)
        auto seg = [&](int s, int& a, int& live) __attribute__((always_inline)) {
          const int i = min(s, cend) - c0;
          if (pre && i < 2) {
            a = half_of(a_pre, i);
            live = half_of(GATED && j == 1 ? live_up : live_pre, i);
          } else {
            a = __builtin_amdgcn_readlane(ta, i);
            live = __builtin_amdgcn_readlane(tl, i);
          }
        };
        int k0, k1;
        auto load = [&](int s, uint16_t* slot, int& rk) __attribute__((always_inline)) {
          int a, live;
          seg(s, a, live);
          load_seg(a, live, slot);
          rk = s <= cend ? min(live - rc, kRankChunk) : 0;
        };
        auto apply = [&](int s, const uint16_t* slot, int rk) __attribute__((always_inline)) {
          uint4 bv[4];
          read_b(slot, bv);
          if (rk <= 0) return;
          const int i = s - c0;
          // the bounds relative to the tile (tile rows and segment bounds are below 2^31)
          apply_seg(__builtin_amdgcn_readlane(tb, i) - (int)p0, __builtin_amdgcn_readlane(te, i) - (int)p0, bv, rk);
        };
        load(c0, slot0, k0);
        if (c0 == s_lo) {
          MLORA_WAIT_VM(4);  // the staged first factors have landed (the sB loads may be in flight)
          lds_sync();
        }
        // (no exit between the halves: a path leaving the loop with one buffer's loads unconsumed made the compiler
        // wait for every load in flight at the top of each iteration, one segment's sB in flight at a time; past
        // the chunk the loads re-read its last segment and rk is 0)
        for (int s = c0; s <= cend; s += 2) {
          load(s + 1, slot1, k1);
          apply(s, slot0, k0);
          load(s + 2, slot0, k0);
          apply(s + 1, slot1, k1);
        }
      }
    };
    if constexpr (GATED) {
      // Gated: gate and up have one capacity c <= 64 (the host checks it), so both matrices' first factors are
      // staged at once and each wave adds only its own matrix's term (waves 0..3 gate, waves 4..7 up). When 2c <= 64
      // the stacked ranks [0, 2c) fit the first buffer (up's from chunk c / 8); otherwise the first buffer holds
      // stacked ranks [0, 64) (gate's c ranks first) and the second stacked ranks [c, c + 64) (up's, from chunk 0).
      // Ranks past a matrix's own c are the other matrix's or the next row's; they are masked by the live rank. The
      // segments' bookkeeping is read per segment (scalar loads, one segment ahead): the lane tables of the plain
      // form, with a wave-dependent matrix, left the compiler short of registers.
      const bool two = L.rank_cap > kRankChunk;
      const int j = wave < 4 ? 0 : 1, capj = L.cap[j];
      lds_sync();  // every wave is done reading the x ring
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        if (h == 1 && !two) break;
#pragma unroll
        for (int i = 0; i < kXLoads; ++i) {
          const int row = (8 * i + wave) * 8 + (lane >> 3);
          const uint32_t off =
              (uint32_t)(((p0 + row) * L.rank_cap + h * L.cap[0] + (swz_slot(row, lane & 7) << 3)) * 2);
          __builtin_amdgcn_raw_ptr_buffer_load_lds(mres, (lds_void*)((h ? st1 : st0) + (8 * i + wave) * 8 * kTK),
                                                   16, off, 0, 0, 0);
        }
      }
      // the lane's staged rows: row mb * 32 + (lane & 31) of the buffer holding its matrix's ranks (st1 for the up
      // waves when 2c > 64, else st0), whose 16-byte chunk c sits in slot c ^ key; the matrix's ranks start at chunk
      // o8 (16 k16 + 8 (lane >> 5) then in chunk o8 + 2 k16 + (lane >> 5) <= 7 for every k16 below the capacity).
      // Both buffers are read and one value kept: a read through a pointer to either buffer is not known to miss the
      // sB slots, and the compiler would wait for every slot load in flight before each such read.
      const bool in1 = j == 1 && two;
      const uint4* mrow0 = reinterpret_cast<const uint4*>(st0) + (lane & 31) * 8;
      const uint4* mrow1 = reinterpret_cast<const uint4*>(st1) + (lane & 31) * 8;
      const int key = ((lane & 31) >> 1) & 7;
      const int cb = (j == 1 && !two ? capj / 8 : 0) + (lane >> 5);
      const int wcj = wc0 - (j ? inter : 0);  // the wave's first column inside its matrix
      __builtin_amdgcn_sched_barrier(0);  // the staging loads are issued before every load below
      // the first factors of row block cmb (its rows 32 cmb + (lane & 31), 64 ranks of the wave's matrix), read from
      // LDS when a segment first touches the block and kept for the next segments (a decode-shaped block holds ~8)
      uint4 av[4];
      int cmb = -1;
      // per chunk of 64 segments, lane tables (lane i: segment c0 + i's adapter, bounds relative to the tile, and
      // live rank of the wave's matrix), then each segment's sB rows one segment ahead of its products
      for (int c0 = s_lo; c0 <= s_hi; c0 += kWave) {
        const int cend = min(c0 + kWave - 1, s_hi);  // the chunk's last segment
        const int sc = min(c0 + lane, cend);
        const int ta = r.seg_adapter[sc];
        const int tb = r.seg_start[sc] - (int)p0, te = r.seg_start[sc + 1] - (int)p0;  // tile rows: below 2^31
        const int tl = ta == 0 ? 0 : live_rank(L, ta, j);
        // segment s's sB rows into a slot, and its live rank `rk` (0 past the chunk: the loads then re-read its last
        // segment's)
        auto load_b = [&](int s, uint16_t* slot, int& rk) __attribute__((always_inline)) {
          const int i = min(s, cend) - c0;
          int a, live;
          if (c0 == s_lo && i < 2) {  // read ahead in the prologue
            a = half_of(a_pre, i);
            live = half_of(j == 0 ? live_pre : live_up, i);
          } else {
            a = __builtin_amdgcn_readlane(ta, i);
            live = __builtin_amdgcn_readlane(tl, i);
          }
          rk = s <= cend ? live : 0;
          stage_b(slot, L.pool + (int64_t)a * L.pool_stride + L.off_b[j], sb_stride(live, capj), 0, wcj, inter);
        };
        // its products, the operands read from the slot, zero past live rank `rk`
        auto apply = [&](int s, const uint16_t* slot, int rk) __attribute__((always_inline)) {
          uint4 bv[4];
          read_b(slot, bv);
          if (rk <= 0) return;
          const int sb = __builtin_amdgcn_readlane(tb, s - c0), se = __builtin_amdgcn_readlane(te, s - c0);
          // products of the 16-rank groups below the live rank; when the live rank is not a multiple of 16, the
          // ranks past it in its last group are zeroed in both operands (the first factors there are not written)
          const int nk = (rk + 15) >> 4;
          const bool ragged = (rk & 15) != 0;
          if (ragged) {
#pragma unroll
            for (int k16 = 0; k16 < 4; ++k16) bv[k16] = keep_first(bv[k16], rk - (16 * k16 + 8 * (lane >> 5)));
          }
#pragma unroll
          for (int mb = 0; mb < MB; ++mb) {
            if (mb * 32 >= se || mb * 32 + 32 <= sb) continue;
            if (cmb != mb) {
#pragma unroll
              for (int k16 = 0; k16 < 4; ++k16) {
                const uint4 a0 = mrow0[mb * 256 + (((cb + 2 * k16) & 7) ^ key)];
                const uint4 a1 = mrow1[mb * 256 + (((cb + 2 * k16) & 7) ^ key)];
                av[k16] = in1 ? a1 : a0;
              }
              cmb = mb;
            }
            const bool rin = mb * 32 + (lane & 31) >= sb && mb * 32 + (lane & 31) < se;
            uint4 v[4];
#pragma unroll
            for (int k16 = 0; k16 < 4; ++k16) v[k16] = rin ? av[k16] : make_uint4(0, 0, 0, 0);
            if (ragged) {
#pragma unroll
              for (int k16 = 0; k16 < 4; ++k16) v[k16] = keep_first(v[k16], rk - (16 * k16 + 8 * (lane >> 5)));
            }
#pragma unroll
            for (int k16 = 0; k16 < 4; ++k16)
              if (k16 < nk) acc[mb] = mfma32(bv[k16], v[k16], acc[mb]);
          }
        };
        int rk0, rk1;
        load_b(c0, slot0, rk0);
        if (c0 == s_lo) {
          MLORA_WAIT_VM(4);  // the first factors have landed (the 4 sB loads may still be in flight)
          lds_sync();
        }
        for (int s = c0; s <= cend; s += 2) {  // (no exit between the halves, as in the plain form)
          load_b(s + 1, slot1, rk1);
          apply(s, slot0, rk0);
          load_b(s + 2, slot0, rk0);
          apply(s + 1, slot1, rk1);
        }
      }
    } else {
      const int jhi = matrix_of(L, min(n0 + kTN, n_out) - 1);
      for (int j = jlo; j <= jhi; ++j) {
        const int oj = col_offset(L, j), cj = L.cols[j], capj = L.cap[j], rho = rank_offset(L, j);
        // the wave's column inside matrix j (others get zero operands)
        const int cc = wc0 + (lane & 31);
        const bool cin = cc >= oj && cc < oj + cj && cc < n_out;
        for (int rc = 0; rc < capj; rc += kRankChunk) {
          // the first factors of row block cmb, read from LDS when a segment first touches the block and kept for the
          // next segments (a decode-shaped block holds ~8)
          uint4 av[4];
          int cmb = -1;
          pass(j, rc, j == jlo,
               // first factors of the tile's rows: 256 rows x 64 ranks, rows of 128 bytes swizzled like x
               [&]() __attribute__((always_inline)) {
                 lds_sync();  // every wave is done with the previous chunk's rows
#pragma unroll
                 for (int i = 0; i < kXLoads; ++i) {
                   const int row = (8 * i + wave) * 8 + (lane >> 3);
                   const uint32_t off =
                       (uint32_t)(((p0 + row) * L.rank_cap + rho + rc + (swz_slot(row, lane & 7) << 3)) * 2);
                   __builtin_amdgcn_raw_ptr_buffer_load_lds(mres, (lds_void*)(st0 + (8 * i + wave) * 8 * kTK), 16,
                                                            off, 0, 0, 0);
                 }
               },
               // the segment's sB rows for ranks rc .. rc + 63 into a slot (the adapter's row stride sbs is at least 8:
               // capj > rc >= 0)
               [&](int a, int live, uint16_t* slot) __attribute__((always_inline)) {
                 stage_b(slot, L.pool + (int64_t)a * L.pool_stride + L.off_b[j], sb_stride(live, capj), rc, wc0 - oj,
                         cj);
               },
               [&](int sb, int se, uint4 (&bv)[4], int rk) __attribute__((always_inline)) {
                 // (sb, se: the segment's bounds relative to the tile's first row; products of the 16-rank groups
                 // below the live rank, the ranks past it in a part-live last group zeroed in both operands)
                 const int nk = (rk + 15) >> 4;
                 const bool ragged = (rk & 15) != 0;
#pragma unroll
                 for (int k16 = 0; k16 < 4; ++k16) bv[k16] = cin ? bv[k16] : make_uint4(0, 0, 0, 0);
                 if (ragged) {
#pragma unroll
                   for (int k16 = 0; k16 < 4; ++k16)
                     if (k16 == nk - 1) bv[k16] = keep_first(bv[k16], rk - (16 * k16 + 8 * (lane >> 5)));
                 }
#pragma unroll
                 for (int mb = 0; mb < MB; ++mb) {
                   if (mb * 32 >= se || mb * 32 + 32 <= sb) continue;
                   const int row = mb * 32 + (lane & 31);
                   if (cmb != mb) {
#pragma unroll
                     for (int k16 = 0; k16 < 4; ++k16) {
                       if (16 * k16 >= capj - rc) break;  // (groups past the capacity are never used)
                       av[k16] = reinterpret_cast<const uint4*>(st0)[swz(row, 2 * k16 + (lane >> 5)) >> 3];
                     }
                     cmb = mb;
                   }
                   const bool rin = row >= sb && row < se;
#pragma unroll
                   for (int k16 = 0; k16 < 4; ++k16) {
                     if (k16 >= nk) break;
                     uint4 v = rin ? av[k16] : make_uint4(0, 0, 0, 0);
                     if (ragged && k16 == nk - 1) v = keep_first(v, rk - (16 * k16 + 8 * (lane >> 5)));
                     acc[mb] = mfma32(bv[k16], v, acc[mb]);
                   }
                 }
               });
        }
      }
    }
    MLORA_WAIT_VM(0);  // the last slot loads (past the last segment) have landed before their buffers are reused
  };
  if (early) {
    lora_term(g_x3, g_x2, g_x0, g_x1);
    lds_sync();  // every wave is done with its sB slots
    dma_x(g_x0, kbase);
    dma_x(g_x1, kbase + min(1, nk - 1) * kTK);
  }
  MLORA_WAIT_VM(kXLoads);  // x(0) has landed
  step_sync();
  load_a(g_x0, 0, a);
  auto run = [&](auto xb, auto wb, int i) __attribute__((always_inline)) {
    constexpr int XB = decltype(xb)::value, WB = decltype(wb)::value;
    const uint16_t* xs = XB == 0 ? g_x0 : XB == 1 ? g_x1 : g_x2;
    const uint16_t* xn = XB == 0 ? g_x1 : XB == 1 ? g_x2 : g_x0;  // buffer (i + 1) % 3
    uint16_t* xf = XB == 0 ? g_x2 : XB == 1 ? g_x0 : g_x1;        // buffer (i + 2) % 3
    WStage& cur = WB == 0 ? s0 : s1;
    WStage& nxt = WB == 0 ? s1 : s0;
    // the next step's words among the first 16 inputs' MFMAs, step i + 2's x rows among the second's
    step(xs, cur, xn, [&]() __attribute__((always_inline)) { fetch_w(nxt, kbase + min(i + 1, nk - 1) * kTK); },
         [&]() __attribute__((always_inline)) { dma_x(xf, kbase + min(i + 2, nk - 1) * kTK); });
  };
  using I0 = std::integral_constant<int, 0>;
  using I1 = std::integral_constant<int, 1>;
  using I2 = std::integral_constant<int, 2>;
  // Whole rounds of six steps in a loop with no other exit (an exit inside the loop made the compiler wait for every
  // load in flight at the top of each round, the x rows two steps ahead included), then the remaining steps.
  const int nfull = nk - nk % 6;
  for (int it = 0; it < nfull; it += 6) {
    run(I0{}, I0{}, it);
    run(I1{}, I1{}, it + 1);
    run(I2{}, I0{}, it + 2);
    run(I0{}, I1{}, it + 3);
    run(I1{}, I0{}, it + 4);
    run(I2{}, I1{}, it + 5);
  }
  if (nfull < nk) {
    run(I0{}, I0{}, nfull);
    if (nfull + 1 < nk) {
      run(I1{}, I1{}, nfull + 1);
      if (nfull + 2 < nk) {
        run(I2{}, I0{}, nfull + 2);
        if (nfull + 3 < nk) {
          run(I0{}, I1{}, nfull + 3);
          if (nfull + 4 < nk) run(I1{}, I0{}, nfull + 4);
        }
      }
    }
  }
  MLORA_WAIT_VM(0);
  lds_sync();

  if (part != nullptr) {
    // Split product: this K range's float32 sums to part[ks][p][c] (sorted rows, `columns` columns per row); the
    // second launch adds the ranges in order, the LoRA term and rounds. Lane l holds four consecutive columns.
    float* pk = part + (int64_t)ks * T * w.columns;
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) {
      const int64_t p = p0 + mb * 32 + (lane & 31);
      if (p >= T) continue;
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int c = n0 + wave * 32 + g * 8 + (lane >> 5) * 4;
        if (c >= w.columns) continue;
        *reinterpret_cast<float4*>(pk + p * w.columns + c) =
            make_float4(acc[mb][4 * g], acc[mb][4 * g + 1], acc[mb][4 * g + 2], acc[mb][4 * g + 3]);
      }
    }
    return;
  }

  if (lora && !early) lora_term(g_x0, g_x1, g_x2, g_x3);

  // Single rounding to bf16 and the stores, through LDS (the whole tile at once): lane l holds, for row
  // mb * 32 + (l & 31), the four consecutive columns 8 g + 4 (l >> 5) .. +3 of its wave's 32 columns; every wave
  // writes its rows to LDS (rows 0..127 in g_x0 and g_x1, rows 128..255 in g_x2 and g_x3, columns 0..127 of the tile
  // in the first of each pair; 256-byte rows with their 16-byte chunks XOR-swizzled by (row & 15)), then every
  // thread reads 16-byte chunks back and writes whole 512-byte tile rows to the token's output row (and to its
  // request's last-token row).
  lds_sync();  // every wave is done reading LDS
#pragma unroll
  for (int half = 0; half < 2; ++half) {
    uint16_t* buf = half == 0 ? ((wave >> 2) ? g_x1 : g_x0) : ((wave >> 2) ? g_x3 : g_x2);
#pragma unroll
    for (int mq = 0; mq < 4; ++mq)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int mb = half * 4 + mq;
        if (mb >= MB) break;  // a 224-row tile's second half has three blocks
        const int row = mq * 32 + (lane & 31);
        const int col = (wave & 3) * 32 + g * 8 + (lane >> 5) * 4;
        const uint32_t lo = pack_bf16x2(acc[mb][4 * g], acc[mb][4 * g + 1]);
        const uint32_t hi = pack_bf16x2(acc[mb][4 * g + 2], acc[mb][4 * g + 3]);
        *reinterpret_cast<uint2*>(&buf[row * 128 + (((col >> 3) ^ (row & 15)) << 3) + (col & 7)]) = make_uint2(lo, hi);
      }
  }
  lds_sync();
  if constexpr (GATED) {
    // gated: 16-byte chunk c of a row's gate columns (first buffer of the pair) with the same chunk of its up columns
    // (second buffer), silu(gate) * up to output columns 128 nt + 8 c .. +7
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int f = tid + kThreads * i;
      const int half = f >> 11, row = (f >> 4) & 127, c = f & 15;
      const int64_t orig = g_orig[half * 128 + row];
      if (orig < 0) continue;
      const int64_t lq = g_last[half * 128 + row];
      const uint16_t* gb = half == 0 ? g_x0 : g_x2;
      const uint16_t* ub = half == 0 ? g_x1 : g_x3;
      const int off = row * 128 + ((c ^ (row & 15)) << 3);
      const uint4 v = silu_mul8(*reinterpret_cast<const uint4*>(&gb[off]), *reinterpret_cast<const uint4*>(&ub[off]));
      const int col = nt * 128 + c * 8;
      if (vec & kStoreVec) {
        if constexpr (EARLY)  // (decode-shaped: non-temporal)
          __builtin_nontemporal_store((u32x4_t){v.x, v.y, v.z, v.w}, reinterpret_cast<u32x4_t*>(y + orig * y_stride + col));
        else
          *reinterpret_cast<uint4*>(y + orig * y_stride + col) = v;
        if (lq >= 0) *reinterpret_cast<uint4*>(last_out + lq * inter + col) = v;
      } else {
        const uint32_t e4[4] = {v.x, v.y, v.z, v.w};
        for (int e = 0; e < 8; ++e) {
          const uint16_t h = (uint16_t)(e4[e >> 1] >> (16 * (e & 1)));
          y[orig * y_stride + col + e] = h;
          if (lq >= 0) last_out[lq * inter + col + e] = h;
        }
      }
    }
    return;
  }
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const int f = tid + kThreads * i;
    const int half = f >> 12, row = (f >> 5) & 127, bsel = (f >> 4) & 1, c = f & 15;
    const int64_t orig = g_orig[half * 128 + row];
    if (orig < 0) continue;
    const int64_t lq = g_last[half * 128 + row];
    const uint16_t* buf = half == 0 ? (bsel ? g_x1 : g_x0) : (bsel ? g_x3 : g_x2);
    uint4 v = *reinterpret_cast<const uint4*>(&buf[row * 128 + ((c ^ (row & 15)) << 3)]);
    const int col = n0 + bsel * 128 + c * 8;
    uint16_t* yr = y + orig * y_stride + col;
    if ((vec & kStoreVec) && col + 7 < n_out) {
      if (vec & kStoreResidual) {  // the output row holds the residual: bf16(residual + output)
        const uint4 rv = *reinterpret_cast<const uint4*>(yr);
        v = make_uint4(add_bf16x2(rv.x, v.x), add_bf16x2(rv.y, v.y), add_bf16x2(rv.z, v.z), add_bf16x2(rv.w, v.w));
      }
      if constexpr (EARLY)  // (decode-shaped: non-temporal)
        __builtin_nontemporal_store((u32x4_t){v.x, v.y, v.z, v.w}, reinterpret_cast<u32x4_t*>(yr));
      else
        *reinterpret_cast<uint4*>(yr) = v;
      if (lq >= 0) *reinterpret_cast<uint4*>(last_out + lq * n_out + col) = v;
    } else {
      const uint32_t e4[4] = {v.x, v.y, v.z, v.w};
      for (int e = 0; e < 8 && col + e < n_out; ++e) {
        uint16_t h = (uint16_t)(e4[e >> 1] >> (16 * (e & 1)));
        if (vec & kStoreResidual) h = add_bf16(yr[e], h);
        yr[e] = h;
        if (lq >= 0) last_out[lq * n_out + col + e] = h;
      }
    }
  }
}

}  // namespace

// Row-tile height for a launch: the one (256 or 224 rows) with the fewer rows per CU over all rounds of tiles, 256 on a
// tie; for decode-shaped passes (`short_segs`: few tokens per adapter segment, where a tile's time goes to streaming
// its segments' sB rather than to its K loop) 128 rows when that is strictly fewer, e.g. 4096 decode rows through
// 2048 columns: 128 tiles of 256 rows leave half the CUs idle. Split launches keep 256 (their range count is sized
// for 256-row tiles).
// The current device's compute units (0 if unknown), read once per device.
static int device_cus() {
  static int cus[64] = {};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 0;
  if (cus[dev] == 0 && hipDeviceGetAttribute(&cus[dev], hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
    cus[dev] = 0;
  return cus[dev] > 0 ? cus[dev] : 0;
}

int tile_blocks(int64_t tokens, int n_tiles, int32_t ksplit, bool short_segs) {
  if (ksplit != 1) return 8;
  const int cus = device_cus();
  if (cus <= 0) return 8;
  auto cost = [&](int mb) {
    const int64_t tiles = ((tokens + 32 * mb - 1) / (32 * mb)) * n_tiles;
    return ((tiles + cus - 1) / cus) * mb;
  };
  const int best = cost(7) < cost(8) ? 7 : 8;
  return short_segs && cost(4) < cost(best) ? 4 : best;
}

int launch_base256(const mlora_int4_t& w, const mlora_lora_t& L, const mlora_route_t& r, const uint16_t* x,
                   int64_t x_stride, uint16_t* y, int64_t y_stride, uint16_t* last_out, int32_t n_out,
                   const uint16_t* mid, float* part, int32_t ksplit, hipStream_t stream, int32_t inter,
                   bool residual) {
  if (residual && (inter > 0 || part != nullptr)) return MLORA_EINVAL;
  if (r.tokens == 0 || n_out == 0) return MLORA_OK;
  if (inter > 0 && (part != nullptr || inter % 128 || n_out != 2 * inter)) return MLORA_EINVAL;
  const int n_tiles = inter > 0 ? inter / 128 : (n_out + kTN - 1) / kTN;
  const int64_t segs = r.requests < L.pool_rows ? r.requests : L.pool_rows;
  const int mb = tile_blocks(r.tokens, n_tiles, ksplit, r.tokens < 16 * (segs > 0 ? segs : 1));
  const int m_tiles = (int)((r.tokens + 32 * mb - 1) / (32 * mb));
  const int64_t blocks = (int64_t)m_tiles * n_tiles * ksplit;
  // 16-byte stores of eight columns need 16-byte aligned output rows
  const bool vec = (reinterpret_cast<uintptr_t>(y) % 16 == 0) && y_stride % 8 == 0 && n_out % 8 == 0 &&
                   (last_out == nullptr || reinterpret_cast<uintptr_t>(last_out) % 16 == 0);  // gated: inter % 128 == 0
  const bool early = part == nullptr && r.tokens < 16 * (segs > 0 ? segs : 1);  // decode-shaped: alternate the order
  const dim3 grid((unsigned)blocks);
  // (224-row tiles have no early form: their scalar registers do not hold both phases' state)
  auto kernel = inter > 0 ? (mb == 4   ? base_mfma256_kernel<4, true, true>
                             : mb == 7 ? base_mfma256_kernel<7, true, false>
                             : early   ? base_mfma256_kernel<8, true, true>
                                       : base_mfma256_kernel<8, true, false>)
                          : (mb == 4   ? base_mfma256_kernel<4, false, true>
                             : mb == 7 ? base_mfma256_kernel<7, false, false>
                             : early   ? base_mfma256_kernel<8, false, true>
                                       : base_mfma256_kernel<8, false, false>);
  hipLaunchKernelGGL(kernel, grid, dim3(kThreads), 0, stream, w, L, r, x, x_stride, y, y_stride, last_out, n_out, mid,
                     n_tiles, (vec ? kStoreVec : 0) | (residual ? kStoreResidual : 0) | (early ? kLoraEarly : 0), part,
                     ksplit, (int32_t)blocks,
                     inter);
  return hipGetLastError() == hipSuccess ? MLORA_OK : MLORA_ELAUNCH;
}
