// The LoRA first factor ("shrink"): mid[p, rho_j + q] = bf16( sum_k x[perm[p], k] A_j[a][q, k] ) for every sorted
// token position p of an adapter segment, matrix j of the group and live rank q. Summed in float32 in a fixed
// order and rounded once to bf16, as the reference rounds its first factor before the second product
// (engine/fast_path.py:159-177,196; engine/int4_kernels.py:67-82,120). Two kernels, chosen by segment length:
//  - shrink_seg: few tokens per adapter (decode). One workgroup per (segment, 32-rank block) streams those 32 rows
//    of A once into MFMA operands, the segment's rows as the other operand; its waves split the inputs and add their
//    sums in a fixed order. Memory-bound on A.
//  - shrink_tile: long segments (prefill). Workgroups per 128 sorted positions, 4 waves of 32 rows; the x rows and
//    the adapter's A rows stream through LDS rings two steps ahead, A shared by the waves; each wave sums its rows
//    over all the inputs in order.
#include <type_traits>

#include "shrink_seg.h"
#include "tile_common.h"

namespace {

using namespace mlora;

constexpr int kSChunk = 64;   // inputs per staged chunk (128-byte rows)

__device__ __forceinline__ void drain_lds() { asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory"); }

template <int RB, int D>
__global__ __launch_bounds__(256) void shrink_tile_kernel(mlora_lora_t L, mlora_route_t r,
                                                          const uint16_t* __restrict__ x, int64_t x_stride, int32_t k,
                                                          uint16_t* __restrict__ mid) {
  constexpr int kRows = 128;
  constexpr int kLoads = 4 + RB;  // memory instructions per lane and step: x rows, then A rows
  static_assert(RB >= 1 && RB <= 4, "at most 4 blocks of A per pass");
  static_assert(D >= 3 && D <= 5, "rings of 3 to 5 slots");
  // rings of D x buffers (128 rows x 64 inputs) and D A buffers (RB blocks of 32 stacked ranks x 64 inputs), distinct
  // arrays so each slot is known at compile time; only the first D of each are used (and allocated). The host picks
  // D for the LDS a workgroup may take: two per CU, or one with more steps in flight.
  __shared__ __attribute__((aligned(16))) uint16_t t_x0[kRows * kSChunk];
  __shared__ __attribute__((aligned(16))) uint16_t t_x1[kRows * kSChunk];
  __shared__ __attribute__((aligned(16))) uint16_t t_x2[kRows * kSChunk];
  __shared__ __attribute__((aligned(16))) uint16_t t_x3[kRows * kSChunk];
  __shared__ __attribute__((aligned(16))) uint16_t t_x4[kRows * kSChunk];
  __shared__ __attribute__((aligned(16))) uint16_t t_a0[RB * 32 * kSChunk];
  __shared__ __attribute__((aligned(16))) uint16_t t_a1[RB * 32 * kSChunk];
  __shared__ __attribute__((aligned(16))) uint16_t t_a2[RB * 32 * kSChunk];
  __shared__ __attribute__((aligned(16))) uint16_t t_a3[RB * 32 * kSChunk];
  __shared__ __attribute__((aligned(16))) uint16_t t_a4[RB * 32 * kSChunk];
  auto xslot = [&](auto slot) __attribute__((always_inline)) {
    constexpr int S = decltype(slot)::value % D;
    if constexpr (S == 0) return t_x0;
    else if constexpr (S == 1) return t_x1;
    else if constexpr (S == 2) return t_x2;
    else if constexpr (S == 3) return t_x3;
    else return t_x4;
  };
  auto aslot = [&](auto slot) __attribute__((always_inline)) {
    constexpr int S = decltype(slot)::value % D;
    if constexpr (S == 0) return t_a0;
    else if constexpr (S == 1) return t_a1;
    else if constexpr (S == 2) return t_a2;
    else if constexpr (S == 3) return t_a3;
    else return t_a4;
  };
  const int64_t T = r.tokens;
  const int64_t p0 = (int64_t)blockIdx.x * kRows;
  if (p0 >= T) return;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int s_first = r.seg_of[p0], s_last = r.seg_of[min(p0 + kRows, T) - 1];
  const int s_lo = blockIdx.y == 0 ? s_first : s_first + 1, s_hi = blockIdx.y == 0 ? s_first : s_last;
  if (s_lo > s_hi) return;
  // x staging: instruction i of wave w fills rows 8 (4 i + w) .. +7; lane l writes 16-byte slot l & 7 of row
  // +(l >> 3), which holds logical chunk swz_slot(row, l & 7). Rows past the tokens read the tile's first row.
  const uint16_t* xsrc[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int row = 8 * (4 * i + wave) + (lane >> 3);
    const int64_t p = p0 + row;
    xsrc[i] = x + (int64_t)r.tok_perm[p < T ? p : p0] * x_stride + 8 * swz_slot(row, lane & 7);
  }
  const int nk = k / kSChunk;
  const int R = L.rank_cap, nblk = (R + 31) / 32;
  const int orow = wave * 32 + (lane & 31);  // the lane's x operand row (and token of its accumulators)
  const int64_t prow = p0 + orow;
  for (int s = s_lo; s <= s_hi; ++s) {
    const int a = r.seg_adapter[s];
    if (a == 0) continue;  // the base row: no first factor is read
    const int64_t sb = r.seg_start[s], se = r.seg_start[s + 1];
    const uint16_t* Abase = L.pool + (int64_t)a * L.pool_stride + L.off_a;
    const int passes = (nblk + RB - 1) / RB;
    for (int pass = 0; pass < passes; ++pass) {
      const int b0 = pass * RB;
      // A staging: instruction i of wave w fills stacked rows 32 b0 + 8 (4 i + w) .. +7 (rows past R re-read row
      // R - 1, never written out)
      // (a fixed-size array: captured by the lambdas below, an array sized by RB kept the compiler from emitting the
      // kernel's host-side launch stubs)
      const uint16_t* asrc[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int row = 8 * (4 * i + wave) + (lane >> 3);
        asrc[i] = Abase + (int64_t)min(32 * b0 + row, R - 1) * k + 8 * swz_slot(row, lane & 7);
      }
      // a step's loads into ring slot (xs, as); past the last step they re-read it (the same number of loads in
      // flight at every wait)
      auto issue = [&](uint16_t* xs, uint16_t* as, int c) __attribute__((always_inline)) {
        const int kc = min(c, nk - 1) * kSChunk;
#pragma unroll
        for (int i = 0; i < 4; ++i)
          __builtin_amdgcn_global_load_lds(xsrc[i] + kc, (lds_void*)(xs + 8 * (4 * i + wave) * kSChunk), 16, 0, 0);
#pragma unroll
        for (int i = 0; i < RB; ++i)
          __builtin_amdgcn_global_load_lds(asrc[i] + kc, (lds_void*)(as + 8 * (4 * i + wave) * kSChunk), 16, 0, 0);
      };
      f32x16_t acc[RB];
#pragma unroll
      for (int bi = 0; bi < RB; ++bi) acc[bi] = f32x16_t{};
      auto compute = [&](const uint16_t* xs, const uint16_t* as) __attribute__((always_inline)) {
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          const int c = 2 * t + (lane >> 5);
          const uint4 xv = *reinterpret_cast<const uint4*>(&xs[swz(orow, c)]);
#pragma unroll
          for (int bi = 0; bi < RB; ++bi) {
            const uint4 av = *reinterpret_cast<const uint4*>(&as[swz(bi * 32 + (lane & 31), c)]);
            acc[bi] = mfma32(av, xv, acc[bi]);
          }
        }
      };
      // Step i reads slot i % D. Its loads landed (the wave's own: at most those of the D - 2 steps after it are in
      // flight), then the barrier (every wave's have, and every wave is done reading step i - 1's slot), then step
      // i + D - 1's loads into that slot, then the MFMAs of step i.
      using I0 = std::integral_constant<int, 0>;
      using I1 = std::integral_constant<int, 1>;
      using I2 = std::integral_constant<int, 2>;
      using I3 = std::integral_constant<int, 3>;
      using I4 = std::integral_constant<int, 4>;
      __syncthreads();  // the previous pass (or segment) is done reading the rings
      issue(xslot(I0{}), aslot(I0{}), 0);
      issue(xslot(I1{}), aslot(I1{}), 1);
      if constexpr (D > 3) issue(xslot(I2{}), aslot(I2{}), 2);
      if constexpr (D > 4) issue(xslot(I3{}), aslot(I3{}), 3);
      auto step = [&](auto slot, int i) __attribute__((always_inline)) {
        constexpr int S = decltype(slot)::value;
        MLORA_WAIT_VM((D - 2) * kLoads);
        __builtin_amdgcn_s_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
        issue(xslot(std::integral_constant<int, S + D - 1>{}), aslot(std::integral_constant<int, S + D - 1>{}),
              i + D - 1);
        compute(xslot(slot), aslot(slot));
        drain_lds();  // this step's LDS reads are done before the next barrier
      };
      for (int i = 0; i < nk; i += D) {
        step(I0{}, i);
        if (i + 1 >= nk) break;
        step(I1{}, i + 1);
        if (i + 2 >= nk) break;
        step(I2{}, i + 2);
        if constexpr (D > 3) {
          if (i + 3 >= nk) break;
          step(I3{}, i + 3);
        }
        if constexpr (D > 4) {
          if (i + 4 >= nk) break;
          step(I4{}, i + 4);
        }
      }
      MLORA_WAIT_VM(0);
      // lane l holds, for token p0 + orow and block bi, stacked ranks 32 (b0 + bi) + 8 g + 4 (l >> 5) + e
      if (prow >= sb && prow < se && prow < T) {
        uint16_t* mrow = mid + prow * R;
#pragma unroll
        for (int bi = 0; bi < RB; ++bi) {
#pragma unroll
          for (int g = 0; g < 4; ++g) {
            const int n0 = 32 * (b0 + bi) + 8 * g + 4 * (lane >> 5);
            if (n0 >= R) continue;
            // the matrix holding rank n0 (capacities are multiples of 8, so the four ranks n0..n0+3 share it)
            int j = 0, rho = 0;
            while (j + 1 < L.n_mats && n0 >= rho + L.cap[j]) rho += L.cap[j++];
            const int live = live_rank(L, a, j) - (n0 - rho);  // ranks n0.. of matrix j below its live rank
            const uint32_t lo = pack_bf16x2(acc[bi][4 * g], acc[bi][4 * g + 1]);
            const uint32_t hi = pack_bf16x2(acc[bi][4 * g + 2], acc[bi][4 * g + 3]);
            if (live >= 4) {
              *reinterpret_cast<uint2*>(mrow + n0) = make_uint2(lo, hi);
            } else {
              const uint16_t h[4] = {(uint16_t)lo, (uint16_t)(lo >> 16), (uint16_t)hi, (uint16_t)(hi >> 16)};
              for (int e = 0; e < live; ++e) mrow[n0 + e] = h[e];
            }
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
  shrink_seg_block(L, r, x, x_stride, k, mid, max_blocks, blockIdx.x, lds, lds + kSegLds / 2);
}

}  // namespace

int launch_shrink(const mlora_lora_t& L, const mlora_route_t& r, const uint16_t* x, int64_t x_stride, int32_t k,
                    uint16_t* mid, bool mfma, hipStream_t stream) {
  if (r.tokens == 0 || r.max_segs == 0) return MLORA_OK;
  if (mfma) {
    // 32-rank blocks of the stacked capacity, in passes of at most 4 (as even as the count allows)
    const int nblk = (L.rank_cap + 31) / 32;
    if (nblk == 0) return MLORA_OK;
    const int passes = (nblk + 3) / 4, rb = (nblk + passes - 1) / passes;
    const dim3 grid((unsigned)((r.tokens + 127) / 128), 2);
    // ring slots: 20 KB a slot at one block (4 slots, two workgroups per CU), 24 KB at two (3 slots, two per CU),
    // 28 and 32 KB at three and four (5 and 4 slots, one per CU)
    if (rb == 1)
      hipLaunchKernelGGL((shrink_tile_kernel<1, 4>), grid, dim3(256), 0, stream, L, r, x, x_stride, k, mid);
    else if (rb == 2)
      hipLaunchKernelGGL((shrink_tile_kernel<2, 3>), grid, dim3(256), 0, stream, L, r, x, x_stride, k, mid);
    else if (rb == 3)
      hipLaunchKernelGGL((shrink_tile_kernel<3, 5>), grid, dim3(256), 0, stream, L, r, x, x_stride, k, mid);
    else
      hipLaunchKernelGGL((shrink_tile_kernel<4, 4>), grid, dim3(256), 0, stream, L, r, x, x_stride, k, mid);
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
