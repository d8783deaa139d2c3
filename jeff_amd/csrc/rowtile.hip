// Row-tile INT4 product for passes of few tokens per adapter segment (decode), any number of tokens:
//   y[perm[p], c] = bf16( sum_k x[perm[p], k] W[c, k] + sum_q mid[p, rho_j + q] sB_j[a(p)][c - o_j, q] )
// A workgroup takes 64 sorted rows (a row tile) by 64 NB columns. Its 4 waves each own all 64 rows and 16 NB columns,
// as 4 x NB blocks of v_mfma_f32_16x16x32_bf16 (the weights the first operand, x rows the second). Lane i of a wave's
// column block nb stands for column NB i + nb of the wave's columns, so a lane loads the NB words of one input octet
// of its NB adjacent columns with one load, and ends with 4 NB adjacent outputs of one row.
// Per 64-input step, P steps ahead: the tile's x rows go into an LDS ring (buffer loads with the LDS flag, read by the
// 4 waves), the step's scales and zero points of the tile's columns into a small LDS ring beside it, each wave's
// packed words straight into its registers; each wave dequantises its own words in registers.
// LoRA: the adapter segments crossing the tile are spread over the K loop's steps, at most one per step. A segment's
// second-factor rows (sB of the wave's columns at the adapter's live rank) load P steps ahead with the step's other
// loads, so their HBM traffic streams beside the base's MFMAs instead of after them. Its term goes into the row blocks
// it crosses, with the first factors of rows outside the segment, and ranks past its live rank, set to zero. Segments
// beyond the steps (more segments than steps: short inputs, many empty requests) are added after the loop.
#include <type_traits>
#include <utility>

#include "tile_common.h"

namespace {

using namespace mlora;

constexpr int kRThreads = 256;        // 4 waves
constexpr int kRRows = 64;            // sorted rows of a tile: 4 blocks of 16
constexpr int kRMB = kRRows / 16;
constexpr int kRX = kRRows * kTK * 2 / (kRThreads * 16);  // x loads per lane and step (16 bytes each)
constexpr int kRScale = 1024;         // bytes of a step's scales (waves 0, 1) and zero points (waves 2, 3)

static_assert(kRX == 2, "x rows of a step: two 16-byte loads per lane");

// The LDS ring: one array per slot (a step's x rows, then its scales and zero points), so that the compiler sees which
// slot each LDS read touches and does not make it wait for the loads in flight into the other slots (loads with the
// LDS flag count as writes to their array; the compiler tells apart at most 8 such arrays).
constexpr int kRSlots = 7;
constexpr int kRSlotBytes = kRRows * kTK * 2 + kRScale;
__shared__ __attribute__((aligned(16))) uint8_t rt_r0[kRSlotBytes], rt_r1[kRSlotBytes], rt_r2[kRSlotBytes],
    rt_r3[kRSlotBytes], rt_r4[kRSlotBytes], rt_r5[kRSlotBytes], rt_r6[kRSlotBytes];
template <int B>
__device__ __forceinline__ uint8_t* ring_slot() {
  static_assert(B >= 0 && B < kRSlots, "ring slot");
  if constexpr (B == 0) return rt_r0;
  else if constexpr (B == 1) return rt_r1;
  else if constexpr (B == 2) return rt_r2;
  else if constexpr (B == 3) return rt_r3;
  else if constexpr (B == 4) return rt_r4;
  else if constexpr (B == 5) return rt_r5;
  else return rt_r6;
}
template <int B>
__device__ __forceinline__ uint16_t* x_slot() { return reinterpret_cast<uint16_t*>(ring_slot<B>()); }
template <int B>
__device__ __forceinline__ uint8_t* s_slot() { return ring_slot<B>() + kRRows * kTK * 2; }

// Column tiles of a product with n_out outputs (gated: inter gate columns) at nb column blocks per wave.
int rowtile_ctiles(int32_t n_out, int32_t inter, int nb) {
  return inter > 0 ? inter / (32 * nb) : (n_out + 64 * nb - 1) / (64 * nb);
}

__device__ __forceinline__ f32x4_t mfma16(uint4 a, uint4 b, f32x4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(a), as_bf16x8(b), c, 0, 0, 0);
}

// NB consecutive words of one input octet (one load)
template <int NB>
struct Words {
  uint32_t v[NB];
};
template <int NB>
__device__ __forceinline__ Words<NB> load_words(__amdgpu_buffer_rsrc_t res, uint32_t voff, uint32_t soff) {
  Words<NB> r;
  if constexpr (NB == 1) {
    r.v[0] = __builtin_amdgcn_raw_buffer_load_b32(res, voff, soff, 0);
  } else if constexpr (NB == 2) {
    const auto t = __builtin_amdgcn_raw_buffer_load_b64(res, voff, soff, 0);
    r.v[0] = t[0];
    r.v[1] = t[1];
  } else if constexpr (NB == 3) {
    const auto t = __builtin_amdgcn_raw_buffer_load_b96(res, voff, soff, 0);
    r.v[0] = t[0];
    r.v[1] = t[1];
    r.v[2] = t[2];
  } else {
    const auto t = __builtin_amdgcn_raw_buffer_load_b128(res, voff, soff, 0);
    r.v[0] = t[0];
    r.v[1] = t[1];
    r.v[2] = t[2];
    r.v[3] = t[3];
  }
  return r;
}

// Steps of loads in flight: 5, or 3 when 5 steps' loads would pass the wave's 6-bit count of outstanding loads (odd,
// so that the ring's P + 1 slots are even in number).
constexpr int rowtile_depth(int nb, int capc) {
  const int per = kRX + 1 + 2 + nb * capc;
  return 5 * per <= 63 ? 5 : 3;
}

template <int... I, class F>
__device__ __forceinline__ void unroll(std::integer_sequence<int, I...>, F&& f) {
  (f(std::integral_constant<int, I>{}), ...);
}

// NB: column blocks of 16 per wave; CAPC: 32-rank chunks of the largest capacity (1 or 2); GATED: the tile's first
// half are gate columns 32 NB ct .. +32 NB, its second half the same up columns, and the output is silu(gate) * up.
template <int NB, int CAPC, bool GATED>
__global__ __launch_bounds__(kRThreads) void rowtile_kernel(mlora_int4_t w, mlora_lora_t L, mlora_route_t r,
                                                            const uint16_t* __restrict__ x, int64_t x_stride,
                                                            uint16_t* __restrict__ y, int64_t y_stride,
                                                            uint16_t* __restrict__ last_out, int32_t n_out,
                                                            const uint16_t* __restrict__ mid, int32_t n_rtiles,
                                                            int32_t n_ctiles, int32_t vec, int32_t inter) {
  constexpr int CT = 64 * NB, CW = 16 * NB, HALF = CT / 2;
  constexpr int P = rowtile_depth(NB, CAPC), S = P + 1;
  constexpr int kSB = NB * CAPC;             // sB loads per lane and step
  constexpr int kPer = kRX + 1 + 2 + kSB;    // loads per lane and step: x rows, scales, two word octets, sB
  static_assert(P * kPer <= 63, "loads in flight beyond the wave's counter");
  static_assert(S <= kRSlots, "ring slots");

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int li = lane & 15, lq = lane >> 4;
  // block -> (column tile ct, row tile rt), row tiles innermost: the row tiles of a column tile share an XCD (its
  // words are read from HBM once and from that XCD's L2 by the others)
  const int b = xcd_tile(blockIdx.x, n_rtiles * n_ctiles);
  const int ct = b / n_rtiles, rt = b - ct * n_rtiles;
  const int T = (int)r.tokens;
  const int p0 = rt * kRRows;
  const int rows = min(kRRows, T - p0);
  const int nk = w.k / kTK;

  // local column lc of the tile -> kernel column
  auto gcol = [&](int lc) { return GATED ? (lc < HALF ? lc : inter - HALF + lc) + HALF * ct : CT * ct + lc; };
  const int wc0 = CW * wave;  // the wave's first local column
  const int gw0 = gcol(wc0);  // and its kernel column

  // x: load i of wave `wave` fills tile rows (2 wave + i) * 8 .. +7; lane l writes LDS chunk slot l & 7 of row
  // +(l >> 3), which holds logical chunk swz_slot(row, l & 7). Rows past the tokens read row 0 of the pass.
  const __amdgpu_buffer_rsrc_t xres =
      __builtin_amdgcn_make_buffer_rsrc((void*)x, (short)0, (int)0xFFFFFFFFu, 0x00020000);
  uint32_t xoff[kRX];
#pragma unroll
  for (int i = 0; i < kRX; ++i) {
    const int row = (kRX * wave + i) * 8 + (lane >> 3);
    const int p = p0 + row;
    xoff[i] = (uint32_t)(((int64_t)r.tok_perm[p < T ? p : 0] * x_stride + (swz_slot(row, lane & 7) << 3)) * 2);
  }

  // scales and zero points of a step: waves 0, 1 load scale dwords d = 64 wave + lane (local columns 2d, 2d + 1),
  // waves 2, 3 zero-point dwords d = 64 (wave - 2) + lane (local columns 4d .. 4d + 3); lanes past the tile's columns
  // load dword 0 again. Symmetric weights (no zero points): waves 2, 3 load scales, unused.
  const int64_t groups = w.k / w.group;
  const int gshift = w.group == 128 ? 7 : 6;
  const bool asym = w.zeros != nullptr;
  const bool zwave = wave >= 2 && asym;
  const __amdgpu_buffer_rsrc_t szres =
      zwave ? __builtin_amdgcn_make_buffer_rsrc((void*)w.zeros, (short)0, (int)(groups * w.columns), 0x00020000)
            : __builtin_amdgcn_make_buffer_rsrc((void*)w.scales, (short)0, (int)(groups * w.columns * 2), 0x00020000);
  uint32_t szoff;
  {
    const int d = 64 * (wave & 1) + lane;
    if (zwave)
      szoff = (uint32_t)gcol(d < CT / 4 ? 4 * d : 0);
    else
      szoff = (uint32_t)gcol(d < CT / 2 ? 2 * d : 0) * 2;
  }

  // words: octet lq of a 32-input slice, the lane's NB adjacent columns
  const __amdgpu_buffer_rsrc_t wres = __builtin_amdgcn_make_buffer_rsrc(
      (void*)w.words, (short)0, (int)((int64_t)(w.k / 8) * w.columns * 4), 0x00020000);
  const uint32_t woff = (uint32_t)((gw0 + NB * li) + lq * w.columns) * 4;

  // the lane's rows: segment, original token, request whose last token it is (loaded now, used later)
  int rseg[kRMB];
  int orig[kRMB], lastr[kRMB];
#pragma unroll
  for (int mb = 0; mb < kRMB; ++mb) {
    const int p = p0 + 16 * mb + li;
    const bool in = p < T;
    rseg[mb] = in ? r.seg_of[p] : -1;
    orig[mb] = in ? r.tok_perm[p] : 0;
    lastr[mb] = (in && last_out != nullptr) ? r.last_of[p] : -1;
  }

  // the wave's matrix, its capacity, stacked-rank and column offsets
  const int j = GATED ? (wave >= 2 ? 1 : 0) : matrix_of(L, gw0);
  const int capj = L.cap[j];
  const int rho = rank_offset(L, j);
  const int oj = GATED ? (wave >= 2 ? inter : 0) : col_offset(L, j);
  const int jc0 = gw0 - oj;  // the wave's first column in matrix j
  const bool lora = mid != nullptr && capj > 0 && gw0 < n_out;
  const uint16_t* bbase = L.pool + L.off_b[j];
  const int brec = L.cols[j] * capj * 2;  // bytes of matrix j's sB block in a pool row

  // segments crossing the tile: s_lo .. s_hi; per 16-row block, the first and last it crosses
  const int s_lo = __builtin_amdgcn_readfirstlane(r.seg_of[p0]);
  const int s_hi = __builtin_amdgcn_readfirstlane(r.seg_of[p0 + rows - 1]);
  const int nseg = s_hi - s_lo + 1;
  int blo[kRMB], bhi[kRMB];
#pragma unroll
  for (int mb = 0; mb < kRMB; ++mb) {
    const int last = rows - 1 - 16 * mb;
    blo[mb] = last >= 0 ? __builtin_amdgcn_readfirstlane(rseg[mb]) : INT_MAX;
    bhi[mb] = last >= 0 ? __builtin_amdgcn_readlane(rseg[mb], min(last, 15)) : -1;
  }
  // the first 64 segments' adapters and live ranks, one per lane
  const int la = s_lo + lane <= s_hi ? r.seg_adapter[s_lo + lane] : 0;
  const int llive = la == 0 ? 0 : live_rank(L, la, j);

  // first factors of the lane's rows, ranks 32 c + 8 lq .. +7 of matrix j, zero past the pass and past the live rank
  // of the row's own adapter (the first factors past it are not written by the first-factor kernels)
  uint4 m[kRMB][CAPC];
#pragma unroll
  for (int mb = 0; mb < kRMB; ++mb) {
    // the live rank of the row's segment: from the segment's lane, or from memory past the first 64 segments
    const int sq = rseg[mb] - s_lo;
    int rrow = __builtin_amdgcn_ds_bpermute((sq & 63) << 2, llive);
    if (rseg[mb] >= 0 && sq >= kWave) {
      const int a = r.seg_adapter[rseg[mb]];
      rrow = a == 0 ? 0 : live_rank(L, a, j);
    }
    if (rseg[mb] < 0) rrow = 0;
#pragma unroll
    for (int c = 0; c < CAPC; ++c) {
      const int p = p0 + 16 * mb + li, q = 32 * c + 8 * lq;
      const uint4 v = (lora && p < T && q < rrow)
                          ? *reinterpret_cast<const uint4*>(mid + (int64_t)p * L.rank_cap + rho + q)
                          : make_uint4(0, 0, 0, 0);
      m[mb][c] = keep_first(v, rrow - q);
    }
  }

  // the segment (index q in s_lo .. s_hi) whose term step i adds: steps spread over the segments, q(i) = i nseg / nk,
  // a segment added at the first step that names it; one segment per step when there are more segments than steps
  auto seg_q = [&](int i) { return nseg <= nk ? (i * nseg) / nk : i; };
  // adapter and live rank of segment index q (wave-uniform)
  // (read back through readfirstlane on both paths: the compiler must see the rank as uniform, or the branches on it
  // become divergent and the MFMAs under them run with part of the wave masked off)
  auto seg_info = [&](int q, int& a, int& rk) {
    if (q < kWave) {
      a = __builtin_amdgcn_readlane(la, q);
      rk = __builtin_amdgcn_readlane(llive, q);
    } else {
      a = __builtin_amdgcn_readfirstlane(r.seg_adapter[s_lo + q]);
      rk = a == 0 ? 0 : live_rank(L, a, j);
    }
    a = __builtin_amdgcn_readfirstlane(a);
    rk = __builtin_amdgcn_readfirstlane(rk);
  };
  // sB operands of segment index q: column jc0 + NB li + nb, ranks 32 c + 8 lq .. +7, clamped to the adapter's
  // stride (the first factors of ranks past the live rank are masked instead); a matrix without capacity, or columns
  // past the matrix, read nothing (zeros from the buffer's bounds)
  int colv[NB];
#pragma unroll
  for (int nb = 0; nb < NB; ++nb) colv[nb] = jc0 + NB * li + nb;
  // Every step issues the same number of sB loads (the waits count them), but a load the term does not use (a step
  // that adds no segment, a rank chunk past the live rank) runs on lane 0 only, so it costs the memory pipeline next
  // to nothing.
  auto load_b = [&](int q, bool add, uint4 (&bv)[kSB], int& rk) __attribute__((always_inline)) {
    int a;
    seg_info(q, a, rk);
    const int sbs = sb_stride(rk, capj);
    const int lg = __builtin_ctz((unsigned)max(sbs, 8));  // sbs: a power of two, at least 8 when capj > 0
    const __amdgpu_buffer_rsrc_t bres = __builtin_amdgcn_make_buffer_rsrc(
        (void*)(bbase + (int64_t)a * L.pool_stride), (short)0, lora ? brec : 0, 0x00020000);
#pragma unroll
    for (int c = 0; c < CAPC; ++c) {
      const int qq = min(32 * c + 8 * lq, sbs - 8);
      const bool used = add && 32 * c < rk;
#pragma unroll
      for (int nb = 0; nb < NB; ++nb)
        if (used || lane == 0)
          bv[nb * CAPC + c] = __builtin_bit_cast(
              uint4, __builtin_amdgcn_raw_buffer_load_b128(bres, (uint32_t)(((colv[nb] << lg) + qq) * 2), 0, 0));
    }
  };
  // the term of segment s (live rank rk) with its sB operands bv, into the row blocks it crosses: the first factors
  // of rows outside the segment, and of ranks past the live rank, are zero
  f32x4_t acc[kRMB][NB];
#pragma unroll
  for (int mb = 0; mb < kRMB; ++mb)
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) acc[mb][nb] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  auto apply = [&](int s, const uint4 (&bv)[kSB], int rk) __attribute__((always_inline)) {
    if (rk <= 0) return;
#pragma unroll
    for (int mb = 0; mb < kRMB; ++mb) {
      if (s < blo[mb] || s > bhi[mb]) continue;
      const uint32_t keep = rseg[mb] == s ? 0xFFFFFFFFu : 0u;  // the row's first factors, else zero
#pragma unroll
      for (int c = 0; c < CAPC; ++c) {
        if (32 * c >= rk) break;
        const uint4 v = m[mb][c];
        const uint4 am = make_uint4(v.x & keep, v.y & keep, v.z & keep, v.w & keep);
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) acc[mb][nb] = mfma16(bv[nb * CAPC + c], am, acc[mb][nb]);
      }
    }
  };

  // the ring: slot B holds step i (i % S == B): its x rows and scales in LDS, its words, sB operands and segment here
  Words<NB> wv[S][2];
  uint4 bq[S][kSB];
  int brk[S], bqi[S];
  int qissued = -1;  // the segment index of the last step issued
  auto issue = [&](auto slot, int i) __attribute__((always_inline)) {
    constexpr int B = decltype(slot)::value;
    const int is = min(i, nk - 1);  // past the last step: the last step's loads again, unused
    const int kc = is * kTK;
#pragma unroll
    for (int u = 0; u < kRX; ++u)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(xres, (lds_void*)(x_slot<B>() + (kRX * wave + u) * 8 * kTK), 16,
                                               xoff[u], kc * 2, 0, 0);
    const int g = kc >> gshift;
    __builtin_amdgcn_raw_ptr_buffer_load_lds(szres, (lds_void*)(s_slot<B>() + 256 * wave), 4, szoff,
                                             zwave ? g * w.columns : g * w.columns * 2, 0, 0);
#pragma unroll
    for (int h = 0; h < 2; ++h) wv[B][h] = load_words<NB>(wres, woff, (uint32_t)((kc / 8 + 4 * h) * w.columns * 4));
    bqi[B] = seg_q(is);
    const bool add = i < nk && bqi[B] < nseg && bqi[B] != qissued;  // this step adds segment bqi[B]'s term
    qissued = i < nk ? bqi[B] : qissued;
    load_b(min(bqi[B], nseg - 1), add, bq[B], brk[B]);
  };
  // a step's MFMA operands, read and dequantised one step ahead of their MFMAs
  struct Ops {
    uint4 xa[2][kRMB];
    uint4 wa[2][NB];
  };
  Ops ops[2];
  auto prepare = [&](auto slot, Ops& o) __attribute__((always_inline)) {
    constexpr int B = decltype(slot)::value;
    const uint8_t* sb = s_slot<B>();
    const uint4* xs = reinterpret_cast<const uint4*>(x_slot<B>());
    float s0[NB], zs[NB];
    uint32_t zb[NB];
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) {  // every read issued before the first use (symmetric: zero points unused)
      const int lc = wc0 + NB * li + nb;
      s0[nb] = bf16_to_f32(*reinterpret_cast<const uint16_t*>(sb + 2 * lc));
      zb[nb] = sb[512 + lc];
    }
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
      for (int mb = 0; mb < kRMB; ++mb) o.xa[h][mb] = xs[swz(16 * mb + li, 4 * h + lq) >> 3];
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) zs[nb] = (asym ? (float)zb[nb] : 8.0f) * s0[nb];
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) o.wa[h][nb] = dequant_word(wv[B][h].v[nb], s0[nb], zs[nb]);
  };
  int qdone = -1;  // the last segment index whose term was added
  auto mma = [&](const Ops& o) __attribute__((always_inline)) {
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
      for (int mb = 0; mb < kRMB; ++mb)
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) acc[mb][nb] = mfma16(o.wa[h][nb], o.xa[h][mb], acc[mb][nb]);
  };
  auto lora_term = [&](auto slot) __attribute__((always_inline)) {
    constexpr int B = decltype(slot)::value;
    const int q = bqi[B];
    if (lora && q < nseg && q != qdone) {
      apply(s_lo + q, bq[B], brk[B]);
      qdone = q;
    }
  };

  static_assert(S % 2 == 0, "the operands' double buffer follows the step's parity");
  unroll(std::make_integer_sequence<int, P>{}, [&](auto slot) { issue(slot, decltype(slot)::value); });
  MLORA_WAIT_VM((P - 1) * kPer);  // step 0's loads have landed
  step_sync();
  prepare(std::integral_constant<int, 0>{}, ops[0]);
  auto step = [&](auto slot, int i) __attribute__((always_inline)) {
    constexpr int B = decltype(slot)::value, E = B & 1;
    MLORA_WAIT_VM((P - 2) * kPer);  // step i + 1's loads have landed (steps i + 2 .. i + P - 1 may be in flight)
    step_sync();                    // every wave's share of step i + 1's LDS rows is visible; step i - 1's slot is free
    issue(std::integral_constant<int, (B + P) % S>{}, i + P);
    // step i's MFMAs, beside step i + 1's operand reads and dequantisation (past the last step: re-reads, unused):
    // the LDS reads first, then each MFMA followed by a share of the dequantisation's vector instructions, so the
    // matrix and vector pipes run together
    __builtin_amdgcn_sched_barrier(0);
    prepare(std::integral_constant<int, (B + 1) % S>{}, ops[E ^ 1]);
    mma(ops[E]);
    __builtin_amdgcn_sched_group_barrier(0x100, 2 * kRMB + 2 * NB, 0);  // LDS reads: x operands, scales, zero points
#pragma unroll
    for (int k = 0; k < 8 * NB; ++k) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // one MFMA
      __builtin_amdgcn_sched_group_barrier(0x002, 6, 0);  // six vector instructions
    }
    // the next step's dequantised words are used here, so the compiler keeps their dequantisation in this step
    // (beside these MFMAs) instead of moving it next to their MFMAs
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) {
        const uint4& v = ops[E ^ 1].wa[h][nb];
        asm volatile("" ::"v"(v.x), "v"(v.y), "v"(v.z), "v"(v.w));
      }
    __builtin_amdgcn_sched_barrier(0);
    lora_term(slot);
  };
  // whole rounds of S steps (one exit only, at a round's end: the compiler's count of the loads in flight at each use
  // then holds on every path), then the last steps
  int it = 0;
  for (; it + S <= nk; it += S)
    unroll(std::make_integer_sequence<int, S>{}, [&](auto slot) { step(slot, it + decltype(slot)::value); });
  unroll(std::make_integer_sequence<int, S - 1>{}, [&](auto slot) {
    if (it + decltype(slot)::value < nk) step(slot, it + decltype(slot)::value);
  });
  MLORA_WAIT_VM(0);

  // segments past the steps
  if (lora) {
    for (int q = nk; q < nseg; ++q) {
      uint4 bv[kSB];
      int rk;
      load_b(q, true, bv, rk);
      apply(s_lo + q, bv, rk);
    }
  }

  // the lane's 4 NB adjacent outputs of row 16 mb + li: value t is acc[mb][t % NB][t / NB]
  auto pair = [&](int mb, int t) __attribute__((always_inline)) {
    return pack_bf16x2(acc[mb][t % NB][t / NB], acc[mb][(t + 1) % NB][(t + 1) / NB]);
  };
  if constexpr (GATED) {
    // gate wave w and up wave w + 2 hold the same columns' gate and up outputs: each gives the other the rounded
    // outputs of two row blocks through LDS (the ring is idle now) and writes silu(gate) * up for its other two, to
    // the gate columns' output positions
    static_assert(kRMB == 4 && 2 * 2 * NB * 64 * 4 <= 4096, "two blocks of a wave's rounded outputs in 4 KB");
    const bool gate = wave < 2;
    uint32_t* ex = reinterpret_cast<uint32_t*>((wave & 1) ? rt_r1 : rt_r0);
    uint32_t* give = ex + (gate ? 1024 : 0);  // gate waves give blocks 2, 3; up waves blocks 0, 1
    const uint32_t* take = ex + (gate ? 0 : 1024);
    auto give_block = [&](auto mbc, int k) __attribute__((always_inline)) {
      constexpr int mb = decltype(mbc)::value;
#pragma unroll
      for (int e = 0; e < 2 * NB; ++e) give[(k * 2 * NB + e) * 64 + lane] = pair(mb, 2 * e);
    };
    auto finish_block = [&](auto mbc, int k) __attribute__((always_inline)) {
      constexpr int mb = decltype(mbc)::value;
      if (16 * mb + li >= rows) return;
      const int64_t o = orig[mb], lr = lastr[mb];
#pragma unroll
      for (int g = 0; g < NB; ++g) {
        const uint2 own = make_uint2(pair(mb, 4 * g), pair(mb, 4 * g + 2));
        const uint2 other = make_uint2(take[(k * 2 * NB + 2 * g) * 64 + lane], take[(k * 2 * NB + 2 * g + 1) * 64 + lane]);
        const uint2 v = gate ? silu_mul4(own, other) : silu_mul4(other, own);
        const int col = HALF * ct + CW * (wave & 1) + 4 * NB * lq + 4 * g;
        store4(y + o * y_stride + col, lr >= 0 ? last_out + lr * inter + col : nullptr, v.x, v.y, inter - col,
               vec & kStoreVec);
      }
    };
    using M0 = std::integral_constant<int, 0>;
    using M1 = std::integral_constant<int, 1>;
    using M2 = std::integral_constant<int, 2>;
    using M3 = std::integral_constant<int, 3>;
    lds_sync();
    if (gate) {
      give_block(M2{}, 0);
      give_block(M3{}, 1);
    } else {
      give_block(M0{}, 0);
      give_block(M1{}, 1);
    }
    lds_sync();
    if (gate) {
      finish_block(M0{}, 0);
      finish_block(M1{}, 1);
    } else {
      finish_block(M2{}, 0);
      finish_block(M3{}, 1);
    }
    return;
  }
#pragma unroll
  for (int mb = 0; mb < kRMB; ++mb) {
    if (16 * mb + li >= rows) continue;
    const int64_t o = orig[mb], lr = lastr[mb];
#pragma unroll
    for (int g = 0; g < NB; ++g) {
      const int col = gw0 + 4 * NB * lq + 4 * g;
      store4(y + o * y_stride + col, lr >= 0 ? last_out + lr * n_out + col : nullptr, pair(mb, 4 * g),
             pair(mb, 4 * g + 2), n_out - col, vec);
    }
  }
}

// Column blocks per wave usable for this group: every wave's columns inside one matrix (the last tile's columns past
// the output are padding, zero weights, never stored), the last tile inside the layout's columns; gated: whole tiles.
bool rowtile_nb_ok(const mlora_int4_t& w, const mlora_lora_t& L, int32_t inter, int nb) {
  if (inter > 0) return L.n_mats == 2 && inter % (32 * nb) == 0;
  for (int j = 0; j + 1 < L.n_mats; ++j)
    if (L.cols[j] % (16 * nb)) return false;
  return (int64_t)rowtile_ctiles(w.out, 0, nb) * 64 * nb <= w.columns;
}

template <int NB, int CAPC>
void rowtile_launch(bool gated, unsigned blocks, hipStream_t stream, const mlora_int4_t& w, const mlora_lora_t& L,
                    const mlora_route_t& r, const uint16_t* x, int64_t x_stride, uint16_t* y, int64_t y_stride,
                    uint16_t* last_out, int32_t n_out, const uint16_t* mid, int32_t n_rtiles, int32_t n_ctiles,
                    int32_t vec, int32_t inter) {
  if (gated)
    hipLaunchKernelGGL((rowtile_kernel<NB, CAPC, true>), dim3(blocks), dim3(kRThreads), 0, stream, w, L, r, x,
                       x_stride, y, y_stride, last_out, n_out, mid, n_rtiles, n_ctiles, vec, inter);
  else
    hipLaunchKernelGGL((rowtile_kernel<NB, CAPC, false>), dim3(blocks), dim3(kRThreads), 0, stream, w, L, r, x,
                       x_stride, y, y_stride, last_out, n_out, mid, n_rtiles, n_ctiles, vec, inter);
}

}  // namespace

// Column blocks per wave (1..3) of a row-tile product of this group, or 0 when the kernel cannot run it: the most
// that still give a workgroup to every CU, else the fewest (the most workgroups).
int rowtile_blocks(const mlora_int4_t& w, const mlora_lora_t& L, int64_t tokens, int32_t inter, int cus) {
  for (int j = 0; j < L.n_mats; ++j)  // capacities of two 32-rank chunks; sB blocks addressed with 32-bit offsets
    if (L.cap[j] > 64 || (int64_t)L.cols[j] * L.cap[j] * 2 >= INT_MAX) return 0;
  const int64_t rtiles = (tokens + kRRows - 1) / kRRows;
  int pick = 0;
  for (int nb = 3; nb >= 1; --nb) {
    if (!rowtile_nb_ok(w, L, inter, nb)) continue;
    const int64_t ctiles = rowtile_ctiles(w.out, inter, nb);
    pick = nb;
    if (rtiles * ctiles >= cus) break;
  }
  return pick;
}

int launch_rowtile(const mlora_int4_t& w, const mlora_lora_t& L, const mlora_route_t& r, const uint16_t* x,
                   int64_t x_stride, uint16_t* y, int64_t y_stride, uint16_t* last_out, int32_t n_out,
                   const uint16_t* mid, int nb, hipStream_t stream, int32_t inter, bool residual) {
  if (r.tokens == 0 || n_out == 0) return MLORA_OK;
  if (nb < 1 || nb > 3 || !rowtile_nb_ok(w, L, inter, nb) || (residual && inter > 0)) return MLORA_EINVAL;
  int maxcap = 0;
  for (int j = 0; j < L.n_mats; ++j) maxcap = L.cap[j] > maxcap ? L.cap[j] : maxcap;
  if (maxcap > 64) return MLORA_EINVAL;
  const int capc = maxcap > 32 ? 2 : 1;
  const int n_rtiles = (int)((r.tokens + kRRows - 1) / kRRows);
  const int n_ctiles = rowtile_ctiles(n_out, inter, nb);
  const int out_cols = inter > 0 ? inter : n_out;  // columns of y and last_out
  // 8-byte stores of four columns need 8-byte aligned output rows
  const int32_t vec = (reinterpret_cast<uintptr_t>(y) % 8 == 0 && y_stride % 4 == 0 &&
                       (last_out == nullptr || (reinterpret_cast<uintptr_t>(last_out) % 8 == 0 && out_cols % 4 == 0))
                           ? kStoreVec
                           : 0) |
                      (residual ? kStoreResidual : 0);
  const bool gated = inter > 0;
  const unsigned blocks = (unsigned)(n_rtiles * n_ctiles);
#define MLORA_ROWTILE(NB, CAPC)                                                                                   \
  rowtile_launch<NB, CAPC>(gated, blocks, stream, w, L, r, x, x_stride, y, y_stride, last_out, n_out, mid, n_rtiles, \
                           n_ctiles, vec, inter)
  if (nb == 1) {
    if (capc == 1) MLORA_ROWTILE(1, 1); else MLORA_ROWTILE(1, 2);
  } else if (nb == 2) {
    if (capc == 1) MLORA_ROWTILE(2, 1); else MLORA_ROWTILE(2, 2);
  } else {
    if (capc == 1) MLORA_ROWTILE(3, 1); else MLORA_ROWTILE(3, 2);
  }
#undef MLORA_ROWTILE
  if (hipGetLastError() != hipSuccess) return MLORA_ELAUNCH;
  return MLORA_OK;
}
