// The LoRA first factor ("shrink"): mid[p, rho_j + q] = bf16( sum_k x[perm[p], k] A_j[a][q, k] ) for every sorted
// token position p of an adapter segment, matrix j of the group and live rank q. Summed in float32 in a fixed
// order and rounded once to bf16, as the reference rounds its first factor before the second product
// (engine/fast_path.py:159-177,196; engine/int4_kernels.py:67-82,120). Two kernels, chosen by segment length:
//  - shrink_seg: few tokens per adapter (decode). One workgroup per (segment, 32-rank block) streams those 32 rows
//    of A once into MFMA operands, the segment's rows as the other operand; its waves split the inputs and add their
//    sums in a fixed order. Memory-bound on A.
//  - shrink_mfma: long segments (prefill). Workgroups per 32 sorted positions; their waves split the inputs, stream
//    the x rows through per-wave LDS rings two chunks ahead and A into registers one chunk ahead, and add their
//    partial sums in a fixed order.
#include "shrink_seg.h"
#include "tile_common.h"

namespace {

using namespace mlora;

constexpr int kSRows = 32;    // sorted rows per workgroup
constexpr int kSWaves = 4;    // waves per workgroup, each a contiguous share of the inputs (two workgroups per CU)
constexpr int kSChunk = 64;   // inputs per staged chunk (128-byte rows)

// Per-wave rings of three x chunks (32 rows x 64 inputs each), distinct arrays so the slot is known at compile time.
__shared__ __attribute__((aligned(16))) uint16_t s_ring0[kSWaves * kSRows * kSChunk];
__shared__ __attribute__((aligned(16))) uint16_t s_ring1[kSWaves * kSRows * kSChunk];
__shared__ __attribute__((aligned(16))) uint16_t s_ring2[kSWaves * kSRows * kSChunk];

// Long segments (prefill): two workgroups per 32 sorted rows, (block, 0) for the block's first adapter segment and
// (block, 1) for the rest (none, unless the block crosses a segment boundary), so a crossing block does not take
// twice as long as the others. A workgroup's 4 waves split the input dimension into chunks of 64. A wave streams its
// chunks of the 32 x rows (gathered through the sorted order) into its own three-slot LDS ring with loads that cover
// whole 128-byte rows, two chunks ahead, and loads the matching A operands into registers one chunk ahead; one
// 32x32x16 MFMA per 32-rank block and 16 inputs, A as the first operand so a lane's accumulators hold four
// consecutive ranks of one token. The four partial sums are added in wave order in LDS and rounded once. Rows
// outside the segment read zero x operands.
// KB: 32-rank blocks per pass (1, 2 or 3, chosen by the host from the group's capacities: all of an adapter's blocks
// in one pass when there are one or three, so no block slot is a masked re-read)
template <int KB>
__global__ __launch_bounds__(kSWaves * 64) void shrink_mfma_kernel(mlora_lora_t L, mlora_route_t r,
                                                                  const uint16_t* __restrict__ x, int64_t x_stride,
                                                                  int32_t k, uint16_t* __restrict__ mid) {
  constexpr int kSLoads = 4 + 4 * KB;  // memory instructions per chunk and lane: x rows to LDS, then A
  const int64_t T = r.tokens;
  const int64_t p0 = (int64_t)blockIdx.x * kSRows;
  if (p0 >= T) return;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int64_t prow = p0 + (lane & 31);
  const int nch = k / kSChunk;
  const int c0 = (wave * nch) / kSWaves, c1 = ((wave + 1) * nch) / kSWaves;  // this wave's chunks
  // x staging: instruction i fills rows 8 i .. 8 i + 7 of the wave's ring slot; lane l writes 16-byte slot l & 7 of
  // row 8 i + (l >> 3), which holds logical chunk swz_slot(row, l & 7)
  const uint16_t* xsrc[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int row = 8 * i + (lane >> 3);
    const int64_t p = p0 + row;
    xsrc[i] = x + (int64_t)r.tok_perm[p < T ? p : p0] * x_stride + 8 * swz_slot(row, lane & 7);
  }
  uint16_t* const ring0 = s_ring0 + wave * kSRows * kSChunk;
  uint16_t* const ring1 = s_ring1 + wave * kSRows * kSChunk;
  uint16_t* const ring2 = s_ring2 + wave * kSRows * kSChunk;
  const int orow = lane & 31;  // the operand row of this lane
  const int s_first = r.seg_of[p0], s_last = r.seg_of[min(p0 + kSRows, T) - 1];
  // workgroup (block, 0) takes the block's first segment, (block, 1) the others, so a block that crosses a segment
  // boundary is not twice as long as the rest
  const int s_lo = blockIdx.y == 0 ? s_first : s_first + 1, s_hi = blockIdx.y == 0 ? s_first : s_last;
  for (int s = s_lo; s <= s_hi; ++s) {
    const int a = r.seg_adapter[s];
    if (a == 0) continue;  // the base row: no first factor is read
    const int64_t sb = r.seg_start[s], se = r.seg_start[s + 1];
    const bool rin = prow >= sb && prow < se;
    int rk[MLORA_MAX_MATS];
    int nblk = 0;
    for (int j = 0; j < L.n_mats; ++j) {
      rk[j] = live_rank(L, a, j);
      nblk += (rk[j] + 31) >> 5;
    }
    const uint16_t* Abase = L.pool + (int64_t)a * L.pool_stride + L.off_a + 8 * (lane >> 5);
    for (int b0 = 0; b0 < nblk; b0 += KB) {
      const uint16_t* asrc[KB];
      bool aok[KB];
#pragma unroll
      for (int bi = 0; bi < KB; ++bi) {
        int j = 0, kb = 0;
        rank_block(rk, L.n_mats, min(b0 + bi, nblk - 1), j, kb);
        const int n = kb * 32 + (lane & 31);
        aok[bi] = b0 + bi < nblk && n < rk[j];
        asrc[bi] = Abase + (int64_t)(rank_offset(L, j) + (aok[bi] ? n : 0)) * k;
      }
      f32x16_t acc[KB];
#pragma unroll
      for (int bi = 0; bi < KB; ++bi) acc[bi] = f32x16_t{};
      // rows outside the segment and rank rows past the live rank multiply as zeros (bit masks, not branches)
      const uint32_t xmask = rin ? 0xFFFFFFFFu : 0u;
      uint32_t amask[KB];
#pragma unroll
      for (int bi = 0; bi < KB; ++bi) amask[bi] = aok[bi] ? 0xFFFFFFFFu : 0u;
      if (c1 > c0) {
        uint4 aq0[4][KB], aq1[4][KB];
        // a chunk's x rows into a ring slot and its A operands into registers; every load is unconditional (chunks
        // past the wave's range re-read its last one), so the counts the waits rely on hold on every path
        auto issue_x = [&](uint16_t* slot, int c) {
          const int kc = min(c, c1 - 1) * kSChunk;
#pragma unroll
          for (int i = 0; i < 4; ++i)
            __builtin_amdgcn_global_load_lds(xsrc[i] + kc, (lds_void*)(slot + i * 8 * kSChunk), 16, 0, 0);
        };
        auto issue_a = [&](uint4 (&aq)[4][KB], int c) {
          const int kc = min(c, c1 - 1) * kSChunk;
#pragma unroll
          for (int t = 0; t < 4; ++t)
#pragma unroll
            for (int bi = 0; bi < KB; ++bi)
              aq[t][bi] = *reinterpret_cast<const uint4*>(asrc[bi] + kc + 16 * t);
        };
        auto compute = [&](const uint16_t* slot, const uint4 (&aq)[4][KB]) {
          uint4 xo[4];  // the chunk's four x operands, read before the first MFMA
#pragma unroll
          for (int t = 0; t < 4; ++t)
            xo[t] = *reinterpret_cast<const uint4*>(&slot[swz(orow, 2 * t + (lane >> 5))]);
#pragma unroll
          for (int t = 0; t < 4; ++t) {
            const uint4 xv = make_uint4(xo[t].x & xmask, xo[t].y & xmask, xo[t].z & xmask, xo[t].w & xmask);
#pragma unroll
            for (int bi = 0; bi < KB; ++bi) {
              const uint4 av = aq[t][bi];
              acc[bi] = mfma32(make_uint4(av.x & amask[bi], av.y & amask[bi], av.z & amask[bi], av.w & amask[bi]), xv,
                               acc[bi]);
            }
          }
        };
        // x rows two chunks ahead (three LDS slots), A operands one chunk ahead (two register sets): the loads are
        // issued x(c + 2), A(c + 1) before chunk c is used, so chunk c has landed when the 4 + 8 loads issued after
        // A(c) are the only ones outstanding
        auto sub = [&](uint16_t* xf, uint4 (&an)[4][KB], const uint16_t* xs, const uint4 (&ac)[4][KB],
                       int c) {
          __builtin_amdgcn_s_waitcnt(0xC07F);  // the previous chunk's LDS reads are done before its slot is refilled
          issue_x(xf, c + 2);
          issue_a(an, c + 1);
          MLORA_WAIT_VM(kSLoads);  // chunk c (x rows and A) has landed
          __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront", "local");
          compute(xs, ac);
        };
        issue_x(ring0, c0);
        issue_x(ring1, c0 + 1);
        issue_a(aq0, c0);
        for (int c = c0; c < c1; c += 6) {
          sub(ring2, aq1, ring0, aq0, c);
          if (c + 1 >= c1) break;
          sub(ring0, aq0, ring1, aq1, c + 1);
          if (c + 2 >= c1) break;
          sub(ring1, aq1, ring2, aq0, c + 2);
          if (c + 3 >= c1) break;
          sub(ring2, aq0, ring0, aq1, c + 3);
          if (c + 4 >= c1) break;
          sub(ring0, aq1, ring1, aq0, c + 4);
          if (c + 5 >= c1) break;
          sub(ring1, aq0, ring2, aq1, c + 5);
        }
        MLORA_WAIT_VM(0);
      }
      // the waves' sums in wave order, one 32-rank block at a time through LDS (the rings are free)
      float* red = reinterpret_cast<float*>(s_ring0);  // [wave][register][lane]
#pragma unroll
      for (int bi = 0; bi < KB; ++bi) {
        __syncthreads();  // every wave is done with the rings (and the previous block's sums)
#pragma unroll
        for (int i = 0; i < 16; ++i) red[(wave * 16 + i) * kWave + lane] = acc[bi][i];
        __syncthreads();
        if (b0 + bi < nblk) {
          int j = 0, kb = 0;
          rank_block(rk, L.n_mats, b0 + bi, j, kb);
          for (int e = tid; e < 16 * kWave; e += kSWaves * kWave) {
            const int i = e / kWave, ln = e % kWave;
            float sum = red[i * kWave + ln];
#pragma unroll
            for (int w = 1; w < kSWaves; ++w) sum += red[(w * 16 + i) * kWave + ln];
            const int n = kb * 32 + (i >> 2) * 8 + (ln >> 5) * 4 + (i & 3);
            const int64_t p = p0 + (ln & 31);
            if (n < rk[j] && p >= sb && p < se) mid[p * L.rank_cap + rank_offset(L, j) + n] = f32_to_bf16(sum);
          }
        }
      }
    }
  }
}

// Short segments (decode): one workgroup per (segment, 32-rank block), the body in shrink_seg.h.
__global__ __launch_bounds__(kDWaves * 64) void shrink_seg_kernel(mlora_lora_t L, mlora_route_t r,
                                                                 const uint16_t* __restrict__ x, int64_t x_stride,
                                                                 int32_t k, uint16_t* __restrict__ mid,
                                                                 int32_t max_blocks) {
  __shared__ __attribute__((aligned(16))) uint16_t lds[kSegLds];
  shrink_seg_block(L, r, x, x_stride, k, mid, max_blocks, blockIdx.x, lds);
}

}  // namespace

int launch_shrink(const mlora_lora_t& L, const mlora_route_t& r, const uint16_t* x, int64_t x_stride, int32_t k,
                    uint16_t* mid, bool mfma, hipStream_t stream) {
  if (r.tokens == 0 || r.max_segs == 0) return MLORA_OK;
  if (mfma) {
    const int64_t blocks = (r.tokens + kSRows - 1) / kSRows;
    // blocks per pass: all of an adapter's blocks when that is one or three (every capacity a multiple of 32), else 2
    int cap_blocks = 0;
    for (int j = 0; j < L.n_mats; ++j) cap_blocks += (L.cap[j] + 31) / 32;
    const dim3 grid((unsigned)blocks, 2);
    if (cap_blocks == 1)
      hipLaunchKernelGGL(shrink_mfma_kernel<1>, grid, dim3(kSWaves * 64), 0, stream, L, r, x, x_stride, k, mid);
    else if (cap_blocks == 3)
      hipLaunchKernelGGL(shrink_mfma_kernel<3>, grid, dim3(kSWaves * 64), 0, stream, L, r, x, x_stride, k, mid);
    else
      hipLaunchKernelGGL(shrink_mfma_kernel<2>, grid, dim3(kSWaves * 64), 0, stream, L, r, x, x_stride, k, mid);
  } else {
    int max_blocks = 0;  // 32-rank blocks of an adapter using every matrix's capacity
    for (int j = 0; j < L.n_mats; ++j) max_blocks += (L.cap[j] + 31) / 32;
    const int64_t blocks = (int64_t)r.max_segs * max_blocks;
    if (blocks == 0) return MLORA_OK;
    hipLaunchKernelGGL(shrink_seg_kernel, dim3((unsigned)blocks), dim3(kDWaves * 64), 0, stream, L, r, x, x_stride, k,
                       mid, max_blocks);
  }
  return hipGetLastError() == hipSuccess ? MLORA_OK : MLORA_ELAUNCH;
}
