// The C ABI (include/jeff_mlora.h): argument checks, then kernel launches on the caller's stream.
// Every check runs on the host, before any launch; nothing here allocates, synchronises or reads device memory, so
// the entry points can be recorded into a HIP graph.
#include <climits>
#include <mutex>

#include "mlora_common.h"

// Device scratch of mlora_int4_linear_noalloc: the first factors, then the float32 partials of a split or narrow
// product. One copy per GPU, held until the process ends. Host code never uses this name as an address: it reads
// each device's address once with hipGetSymbolAddress (noalloc_scratch) and passes that pointer to the kernels.
static __device__ __align__(256) uint8_t scratch[MLORA_NOALLOC_SCRATCH_BYTES];

namespace {

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

int check_route(const mlora_route_t* r) {
  if (r == nullptr || r->tokens < 0 || r->requests < 0 || r->max_segs < 0) return MLORA_EINVAL;
  if (r->tokens >= INT_MAX) return MLORA_EOVERFLOW;
  if (r->requests > MLORA_MAX_REQUESTS) return MLORA_EUNSUPPORTED;
  if (r->num_segs == nullptr || r->seg_start == nullptr || r->seg_adapter == nullptr || r->status == nullptr)
    return MLORA_EINVAL;
  if (r->tokens > 0 && (r->tok_perm == nullptr || r->last_of == nullptr || r->seg_of == nullptr)) return MLORA_EINVAL;
  if (r->requests > 0 && r->req_order == nullptr) return MLORA_EINVAL;
  return MLORA_OK;
}

int check_lora(const mlora_lora_t* L, int32_t k, int32_t n_out) {
  if (L == nullptr || L->pool == nullptr || L->ranks == nullptr) return MLORA_EINVAL;
  if (k <= 0 || k % 64) return MLORA_EINVAL;  // the kernels stage x in chunks of 64 inputs
  if (L->n_mats < 1 || L->n_mats > MLORA_MAX_MATS) return MLORA_EUNSUPPORTED;
  if (L->pool_rows < 1 || L->pool_rows > MLORA_MAX_POOL_ROWS || L->ranks_stride < L->n_mats) return MLORA_EINVAL;
  if (!aligned16(L->pool) || L->pool_stride % 8 || L->off_a % 8 || L->off_a < 0) return MLORA_EALIGN;
  if (L->pool_stride < 0) return MLORA_EINVAL;
  int64_t caps = 0, cols = 0;
  for (int j = 0; j < L->n_mats; ++j) {
    if (L->cap[j] < 0 || L->cols[j] <= 0) return MLORA_EINVAL;
    if (L->cap[j] % 8 || L->off_b[j] % 8 || L->off_b[j] < 0) return MLORA_EALIGN;
    // off_b + cols * cap <= pool_stride, without overflow (cols * cap < 2^62)
    if (L->off_b[j] > L->pool_stride || (int64_t)L->cols[j] * L->cap[j] > L->pool_stride - L->off_b[j])
      return MLORA_EINVAL;
    caps += L->cap[j];
    cols += L->cols[j];
  }
  if (caps != L->rank_cap || cols != n_out) return MLORA_EINVAL;
  // off_a + caps * k <= pool_stride (caps < 2^34, k < 2^31: the product is formed only when it fits)
  if (L->off_a > L->pool_stride || (caps > 0 && (L->pool_stride - L->off_a) / caps < k)) return MLORA_EINVAL;
  return MLORA_OK;
}

int check_int4(const mlora_int4_t* w) {
  if (w == nullptr || w->words == nullptr || w->scales == nullptr) return MLORA_EINVAL;
  if (w->group != 64 && w->group != 128) return MLORA_EUNSUPPORTED;
  if (w->k <= 0 || w->k % w->group || w->columns <= 0 || w->columns % 64 || w->out <= 0 || w->out > w->columns)
    return MLORA_EINVAL;
  if (!aligned16(w->words)) return MLORA_EALIGN;
  if ((int64_t)(w->k / 8) * w->columns >= INT_MAX) return MLORA_EOVERFLOW;
  return MLORA_OK;
}

int check_rows(const void* p, int64_t stride, int32_t width) {
  if (p == nullptr || stride < width) return MLORA_EINVAL;
  if (!aligned16(p) || stride % 8) return MLORA_EALIGN;
  return MLORA_OK;
}

// The first factors (tokens x rank_cap bf16) are addressed with 32-bit buffer offsets.
int check_first_factors(const mlora_route_t* r, const mlora_lora_t* L) {
  return r->tokens * (int64_t)L->rank_cap * 2 >= ((int64_t)1 << 31) ? MLORA_EOVERFLOW : MLORA_OK;
}

// Long segments on average (prefill): at least 16 tokens per adapter segment.
bool long_segments(const mlora_route_t* r, int32_t pool_rows) {
  const int64_t segs = r->requests < pool_rows ? r->requests : pool_rows;
  return r->tokens >= 16 * (segs > 0 ? segs : 1);
}

bool shrink_on_mfma(const mlora_route_t* r, int32_t pool_rows, int32_t flags) {
  if (flags & MLORA_FORCE_SHRINK_MFMA) return true;
  if (flags & MLORA_FORCE_SHRINK_SEGMENT) return false;
  return long_segments(r, pool_rows);
}

enum class Base { gemv, fused, split, narrow };

constexpr int64_t kNarrowMaxTokens = 256;  // the narrow kernel's row tile holds every token of the pass
constexpr int64_t kSplitMaxTokens = 1024;  // short-segment passes of this many tokens or more take the fused tiles

// The split product runs the 256 x 256 kernel (32-bit x offsets) and stages first factors of at most
// MLORA_SPLIT_MAX_RANK stacked ranks.
bool split_fits(const mlora_int4_t* w, const mlora_lora_t* L, const mlora_route_t* r, int64_t x_stride) {
  const int64_t row = x_stride > w->k ? x_stride : w->k;  // tokens < 2^31 (check_route): compare by division
  return L->rank_cap <= MLORA_SPLIT_MAX_RANK && (r->tokens == 0 || row < ((int64_t)1 << 31) / r->tokens);
}

// Which base kernels run; EUNSUPPORTED when the flags force one that cannot (forced input ranges: a count of 1, 2,
// 4 or 8 dividing the 64-input steps, for a narrow product only).
// The gated epilogue (MLORA_EPILOGUE_SILU_MUL): 0 when off, else the width of each half (gate, up).
int32_t gated_width(const mlora_int4_t* w, int32_t flags) {
  return (flags & MLORA_EPILOGUE_SILU_MUL) ? w->out / 2 : 0;
}
// The residual epilogue (MLORA_EPILOGUE_RESIDUAL): y holds the residual and receives residual + output.
bool residual_of(int32_t flags) { return (flags & MLORA_EPILOGUE_RESIDUAL) != 0; }

// CUs of the current device (256 when it cannot be asked, e.g. on a host without a GPU).
int device_cus() {
  static int cus[64] = {};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (cus[dev] == 0 && (hipDeviceGetAttribute(&cus[dev], hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
                        cus[dev] <= 0))
    cus[dev] = 256;
  return cus[dev];
}

int base_of(const mlora_int4_t* w, const mlora_lora_t* L, const mlora_route_t* r, int64_t x_stride, int32_t flags,
            Base* out) {
  const bool gated = (flags & MLORA_EPILOGUE_SILU_MUL) != 0, resid = residual_of(flags);
  if (gated && resid) return MLORA_EINVAL;  // one epilogue per product
  const int32_t fs = (flags >> 8) & 0xF;
  if (fs != 0 && (!(fs == 1 || fs == 2 || fs == 4 || fs == 8) || (w->k / 64) % fs)) return MLORA_EUNSUPPORTED;
  if (flags & MLORA_FORCE_BASE_GEMV) {
    if (r->tokens > 8) return MLORA_EUNSUPPORTED;
    *out = Base::gemv;
  } else if (flags & MLORA_FORCE_BASE_SPLIT) {
    if (!split_fits(w, L, r, x_stride)) return MLORA_EUNSUPPORTED;
    *out = Base::split;
  } else if (flags & MLORA_FORCE_BASE_NARROW) {
    if (r->tokens > kNarrowMaxTokens || !split_fits(w, L, r, x_stride)) return MLORA_EUNSUPPORTED;
    *out = Base::narrow;
  } else if (flags & MLORA_FORCE_BASE_MFMA) {
    *out = Base::fused;
  } else if (r->tokens <= 8 && !gated && !resid) {  // (the GEMV kernel has no epilogues: few tokens take the tiles)
    *out = Base::gemv;
  } else if (long_segments(r, L->pool_rows) || !split_fits(w, L, r, x_stride)) {
    *out = Base::fused;
  } else if (r->tokens <= kNarrowMaxTokens) {
    *out = Base::narrow;
  } else {
    // short segments, more tokens: from kSplitMaxTokens on, the 256 x 256 tiles with the LoRA term fused (each
    // segment's bookkeeping from lane tables) beat the split product, whose float32 partials make a round trip
    // through memory
    *out = r->tokens < kSplitMaxTokens ? Base::split : Base::fused;
  }
  if (fs != 0 && *out != Base::narrow) return MLORA_EUNSUPPORTED;
  if (gated) {
    // gate and up of equal width, a multiple of 128 (the tiles pair 128 gate columns with the same up columns);
    // the 256 x 256 kernel for the fused product (32-bit x offsets), the register form of the split epilogue
    const int64_t inter = w->out / 2;
    if (*out == Base::gemv || L->n_mats != 2 || w->out % 256 || L->cols[0] != inter || L->cols[1] != inter ||
        L->cap[0] != L->cap[1] || L->cap[0] > 64)
      return MLORA_EUNSUPPORTED;
    const int64_t row = x_stride > w->k ? x_stride : w->k;
    if (*out == Base::fused && r->tokens > 0 && row >= ((int64_t)1 << 31) / r->tokens) return MLORA_EUNSUPPORTED;
    if (*out == Base::split && !finish_registers(*L)) return MLORA_EUNSUPPORTED;
  }
  if (resid) {
    // the 256 x 256 kernel for the fused product, the register form of the split epilogue
    const int64_t row = x_stride > w->k ? x_stride : w->k;
    if (*out == Base::gemv) return MLORA_EUNSUPPORTED;
    if (*out == Base::fused && r->tokens > 0 && row >= ((int64_t)1 << 31) / r->tokens) return MLORA_EUNSUPPORTED;
    if (*out == Base::split && !finish_registers(*L)) return MLORA_EUNSUPPORTED;
  }
  return MLORA_OK;
}


// Input ranges of a narrow product: the forced count, else the count S in {1, 2, 4, 8} (dividing the 64-input steps)
// with the least estimated time. A base workgroup takes about 0.6 us per step plus 12 us of fixed work, in rounds of
// one per CU. One range: the first factors' own launch before it (~9 us). S ranges: the expand launch after it
// (~9 us) and the float32 ranges' round trip through memory, counted at 1 TB/s (the expand's reads of more ranges
// lengthen its chain). (Fitted to 256-token products of 2048 -> 4096, 2048 -> 2048, gated
// 2048 -> 2 x 6144 and 6144 -> 2048 columns over 1, 2, 4 and 8 ranges; the estimate picks the fastest count of each:
// 2, 4, 1 and 4.)
int32_t narrow_ranges(const mlora_int4_t* w, int32_t flags) {
  if ((flags >> 8) & 0xF) return (flags >> 8) & 0xF;  // forced (base_of checked it)
  const int64_t tiles = w->columns / 64, steps = w->k / 64, cus = device_cus();
  double best = 0.0;
  int32_t pick = 1;
  for (int32_t s = 1; s <= 8; s *= 2) {
    if (steps % s) continue;
    const int64_t rounds = (tiles * s + cus - 1) / cus;
    const double t = (double)rounds * (0.6 * (double)(steps / s) + 12.0) + 9.0 +
                     (double)dec_partials_bytes(*w, s) / 1.0e6;
    if (s == 1 || t < best) {
      best = t;
      pick = s;
    }
  }
  return pick;
}

// Input ranges of a split product: the most (at most 8, each of at least 4 steps of 64 inputs, dividing the steps)
// that keep the first launch within one workgroup per CU (256).
int32_t split_ranges(const mlora_int4_t* w, int64_t tokens) {
  const int64_t tiles = ((tokens + 255) / 256) * ((w->out + 255) / 256);
  const int steps = w->k / 64;
  int best = 1;
  for (int s = 2; s <= 8; ++s)
    if (steps % s == 0 && steps / s >= 4 && tiles * s <= 256) best = s;
  return best;
}

size_t split_bytes(const mlora_int4_t* w, int64_t tokens) {
  return ((size_t)split_ranges(w, tokens) * (size_t)tokens * (size_t)w->columns * 4 + 255) & ~(size_t)255;
}

// Float32 partial bytes the base kernels `base` read and write for this product (0 for the fused kernels).
size_t partials_of(const mlora_int4_t* w, const mlora_route_t* r, Base base, int32_t flags) {
  if (base == Base::narrow) return dec_partials_bytes(*w, narrow_ranges(w, flags));
  return base == Base::split ? split_bytes(w, r->tokens) : 0;
}

// The base product and the LoRA second factor once mid holds the first factors, or, for a narrow product with
// fuse_shrink, as it computes them (its base launch writes mid).
int run_base(const mlora_int4_t* w, const mlora_lora_t* L, const mlora_route_t* r, const uint16_t* x,
             int64_t x_stride, uint16_t* y, int64_t y_stride, uint16_t* last_out, uint16_t* mid, bool fuse_shrink,
             void* partials, size_t partials_bytes, Base base, int32_t flags, hipStream_t s) {
  const int32_t inter = gated_width(w, flags);
  const bool resid = residual_of(flags);
  if (base == Base::narrow) {
    const int32_t ks = narrow_ranges(w, flags);
    const size_t need = dec_partials_bytes(*w, ks);
    if (need > 0 && (partials == nullptr || !aligned16(partials) || partials_bytes < need)) return MLORA_EWORKSPACE;
    return launch_dec(*w, *L, *r, x, x_stride, y, y_stride, last_out, w->out, mid, fuse_shrink,
                      static_cast<float*>(partials), ks, s, inter, resid);
  }
  if (base == Base::fused && (inter > 0 || resid))
    return launch_base256(*w, *L, *r, x, x_stride, y, y_stride, last_out, w->out, mid, nullptr, 1, s, inter, resid);
  if (base != Base::split)
    return launch_base(w, *L, *r, x, x_stride, y, y_stride, last_out, w->out, mid, base == Base::gemv, s);
  if (partials == nullptr || !aligned16(partials) || partials_bytes < split_bytes(w, r->tokens))
    return MLORA_EWORKSPACE;
  const int32_t ks = split_ranges(w, r->tokens);
  float* part = static_cast<float*>(partials);
  int rc = launch_base256(*w, *L, *r, x, x_stride, nullptr, 0, nullptr, w->out, nullptr, part, ks, s);
  if (rc) return rc;
  return launch_finish(*L, *r, part, ks, w->columns, mid, y, y_stride, last_out, w->out, s, inter, resid);
}

// The device address of `scratch` on the current device, looked up once per device (with that device current);
// nullptr when HIP cannot give it.
constexpr int kMaxDevices = 64;
uint8_t* g_scratch[kMaxDevices] = {};
std::once_flag g_scratch_once[kMaxDevices];

uint8_t* noalloc_scratch() {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return nullptr;
  std::call_once(g_scratch_once[dev], [dev] {
    void* p = nullptr;
    if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) == hipSuccess) g_scratch[dev] = static_cast<uint8_t*>(p);
  });
  return g_scratch[dev];
}

}  // namespace

#pragma GCC visibility push(default)
extern "C" {

int mlora_abi_version(void) { return MLORA_ABI_VERSION; }

int mlora_capture_id(void* stream, uint64_t* id) {
  if (id == nullptr) return MLORA_EINVAL;
  hipStreamCaptureStatus status = hipStreamCaptureStatusNone;
  unsigned long long cid = 0;
  if (hipStreamGetCaptureInfo(static_cast<hipStream_t>(stream), &status, &cid) != hipSuccess) return MLORA_ELAUNCH;
  *id = status == hipStreamCaptureStatusActive ? (uint64_t)cid : 0;
  return MLORA_OK;
}

size_t mlora_workspace_bytes(int64_t tokens, int32_t rank_cap) {
  if (tokens <= 0 || rank_cap <= 0) return 256;
  return ((size_t)tokens * (size_t)rank_cap * 2 + 255) & ~(size_t)255;
}

int mlora_route(const int32_t* adp, const int32_t* cu_seqlens, int32_t row_len, const mlora_route_t* route,
                int32_t pool_rows, void* stream) {
  int rc = check_route(route);
  if (rc) return rc;
  if (pool_rows < 1 || pool_rows > MLORA_MAX_POOL_ROWS) return MLORA_EINVAL;
  if (route->requests > 0 && adp == nullptr) return MLORA_EINVAL;
  const int32_t need = route->requests < pool_rows ? route->requests : pool_rows;
  if (route->max_segs < need || (route->requests > 0 && route->max_segs < 1)) return MLORA_EINVAL;
  if (cu_seqlens == nullptr && (row_len < 0 || (int64_t)route->requests * row_len != route->tokens))
    return MLORA_EINVAL;
  return launch_route(adp, cu_seqlens, row_len, *route, pool_rows, static_cast<hipStream_t>(stream));
}

int mlora_int4_plan(int32_t k, int32_t columns, int32_t out, int64_t tokens, int32_t requests, int32_t pool_rows,
                    int32_t rank_cap, int32_t flags, int32_t* base, int32_t* shrink, int32_t* ranges) {
  if (base == nullptr || shrink == nullptr || ranges == nullptr) return MLORA_EINVAL;
  if (k <= 0 || k % 64 || columns <= 0 || columns % 64 || out <= 0 || out > columns || tokens <= 0 || requests < 0 ||
      pool_rows < 1 || rank_cap < 0)
    return MLORA_EINVAL;
  if (tokens >= INT_MAX || (int64_t)(k / 8) * columns >= INT_MAX) return MLORA_EOVERFLOW;  // as the products refuse
  if (requests > MLORA_MAX_REQUESTS) return MLORA_EUNSUPPORTED;
  // descriptors holding only what the rule reads
  const mlora_int4_t w = {nullptr, nullptr, nullptr, k, columns, out, 64};
  mlora_lora_t L = {};
  L.pool_rows = pool_rows;
  L.rank_cap = rank_cap;
  if (flags & MLORA_EPILOGUE_SILU_MUL) {  // a gate_up group: two halves of out / 2, capacities of the register form
    L.n_mats = 2;
    L.cols[0] = L.cols[1] = out / 2;
    L.cap[0] = L.cap[1] = 8;
  } else {  // one matrix of the group's width
    L.n_mats = 1;
    L.cols[0] = out;
  }
  mlora_route_t r = {};
  r.tokens = tokens;
  r.requests = requests;
  Base b;
  const int rc = base_of(&w, &L, &r, k, flags, &b);
  if (rc) return rc;
  *base = b == Base::gemv ? 0 : b == Base::fused ? 1 : b == Base::split ? 2 : 3;
  *shrink = shrink_on_mfma(&r, pool_rows, flags) ? 1 : 0;
  *ranges = b == Base::narrow ? narrow_ranges(&w, flags) : b == Base::split ? split_ranges(&w, tokens) : 1;
  return MLORA_OK;
}

int mlora_dequant(const mlora_int4_t* w, uint16_t* out, void* stream) {
  int rc = check_int4(w);
  if (rc) return rc;
  if (out == nullptr) return MLORA_EINVAL;
  if (!aligned16(out) || w->k % 8) return MLORA_EALIGN;
  return launch_dequant(*w, out, static_cast<hipStream_t>(stream));
}

int mlora_shrink(const mlora_lora_t* lora, const mlora_route_t* route, const uint16_t* x, int64_t x_stride,
                 int32_t k, uint16_t* mid, int32_t flags, void* stream) {
  int rc = check_route(route);
  if (rc) return rc;
  if (lora == nullptr || k <= 0 || k % 64) return MLORA_EINVAL;
  int32_t n_out = 0;
  for (int j = 0; j < lora->n_mats && j < MLORA_MAX_MATS; ++j) n_out += lora->cols[j];
  if ((rc = check_lora(lora, k, n_out)) || (rc = check_first_factors(route, lora))) return rc;
  if (route->tokens == 0) return MLORA_OK;
  if ((rc = check_rows(x, x_stride, k))) return rc;
  if (mid == nullptr) return MLORA_EINVAL;
  return launch_shrink(*lora, *route, x, x_stride, k, mid, shrink_on_mfma(route, lora->pool_rows, flags),
                       static_cast<hipStream_t>(stream));
}

size_t mlora_int4_partials_bytes(const mlora_int4_t* w, const mlora_lora_t* lora, const mlora_route_t* route,
                                 int32_t flags) {
  if (check_int4(w) || check_route(route) || check_lora(lora, w->k, w->out) || route->tokens == 0) return 0;
  Base base;
  if (base_of(w, lora, route, w->k, flags, &base)) return 0;
  return partials_of(w, route, base, flags);
}

size_t mlora_int4_partials_bound(int32_t k, int32_t columns, int32_t out, int64_t tokens) {
  if (k <= 0 || k % 64 || columns <= 0 || columns % 64 || out <= 0 || out > columns || tokens <= 0 ||
      tokens >= INT_MAX)
    return 0;
  const mlora_int4_t w = {nullptr, nullptr, nullptr, k, columns, out, 64};
  // a narrow product (at most kNarrowMaxTokens tokens) at the automatic range count
  size_t most = dec_partials_bytes(w, narrow_ranges(&w, 0));
  // a split product of t <= tokens tokens (more than kNarrowMaxTokens unless forced): within each 256-token band of
  // row tiles the range count is fixed, so the band's last token count needs the most; once a band runs one range
  // the bytes only grow with t, so the last is `tokens` itself
  for (int64_t m = 1; 256 * (m - 1) < tokens; ++m) {
    const int64_t t = 256 * m < tokens ? 256 * m : tokens;
    const size_t b = split_bytes(&w, t);
    most = b > most ? b : most;
    if (split_ranges(&w, t) == 1) {
      const size_t last = split_bytes(&w, tokens);
      most = last > most ? last : most;
      break;
    }
  }
  return most;
}

int mlora_int4_linear(const mlora_int4_t* w, const mlora_lora_t* lora, const mlora_route_t* route,
                      const uint16_t* x, int64_t x_stride, uint16_t* y, int64_t y_stride, uint16_t* last_out,
                      void* workspace, size_t workspace_bytes, void* partials, size_t partials_bytes, int32_t flags,
                      void* stream) {
  int rc = check_int4(w);
  if (rc) return rc;
  if ((rc = check_route(route)) || (rc = check_lora(lora, w->k, w->out)) || (rc = check_first_factors(route, lora)))
    return rc;
  if (route->tokens == 0) return MLORA_OK;
  if ((rc = check_rows(x, x_stride, w->k))) return rc;
  if (y == nullptr || y_stride < (gated_width(w, flags) ? w->out / 2 : w->out)) return MLORA_EINVAL;
  if (workspace == nullptr || !aligned16(workspace)) return MLORA_EWORKSPACE;
  if (workspace_bytes < mlora_workspace_bytes(route->tokens, lora->rank_cap)) return MLORA_EWORKSPACE;
  Base base;
  if ((rc = base_of(w, lora, route, x_stride, flags, &base))) return rc;
  if (base == Base::split && (partials == nullptr || partials_bytes < split_bytes(w, route->tokens)))
    return MLORA_EWORKSPACE;
  hipStream_t s = static_cast<hipStream_t>(stream);
  uint16_t* mid = static_cast<uint16_t*>(workspace);
  const bool mfma_shrink = shrink_on_mfma(route, lora->pool_rows, flags);
  if (base == Base::split && !mfma_shrink) {
    // split product of short segments: the first factor (its own launch: two of its workgroups fit a CU, where the
    // base launch's LDS leaves room for one), the base ranges, then the epilogue
    const int32_t ks = split_ranges(w, route->tokens);
    float* part = static_cast<float*>(partials);
    if ((rc = launch_shrink(*lora, *route, x, x_stride, w->k, mid, false, s))) return rc;
    if ((rc = launch_base256(*w, *lora, *route, x, x_stride, nullptr, 0, nullptr, w->out, nullptr, part, ks, s)))
      return rc;
    return launch_finish(*lora, *route, part, ks, w->columns, mid, y, y_stride, last_out, w->out, s,
                         gated_width(w, flags), residual_of(flags));
  }
  if (base == Base::split) {
    // split product of long segments (forced): the first factor, the base ranges, then the epilogue
    const int32_t ks = split_ranges(w, route->tokens);
    float* part = static_cast<float*>(partials);
    if ((rc = launch_shrink(*lora, *route, x, x_stride, w->k, mid, mfma_shrink, s))) return rc;
    if ((rc = launch_base256(*w, *lora, *route, x, x_stride, nullptr, 0, nullptr, w->out, nullptr, part, ks, s)))
      return rc;
    return launch_finish(*lora, *route, part, ks, w->columns, mid, y, y_stride, last_out, w->out, s,
                         gated_width(w, flags), residual_of(flags));
  }
  if (base == Base::narrow && !mfma_shrink)  // the segment-form first factors inside the base launch
    return run_base(w, lora, route, x, x_stride, y, y_stride, last_out, mid, true, partials, partials_bytes, base,
                    flags, s);
  if ((rc = launch_shrink(*lora, *route, x, x_stride, w->k, mid, mfma_shrink, s))) return rc;
  return run_base(w, lora, route, x, x_stride, y, y_stride, last_out, mid, false, partials, partials_bytes, base,
                  flags, s);
}

int mlora_int4_linear_noalloc(const mlora_int4_t* w, const mlora_lora_t* lora, const mlora_route_t* route,
                              const uint16_t* x, int64_t x_stride, uint16_t* y, int64_t y_stride, uint16_t* last_out,
                              int32_t flags, void* stream) {
  int rc = check_int4(w);
  if (rc) return rc;
  if ((rc = check_route(route)) || (rc = check_lora(lora, w->k, w->out)) || (rc = check_first_factors(route, lora)))
    return rc;
  if (route->tokens == 0) return MLORA_OK;
  Base base;
  if ((rc = base_of(w, lora, route, x_stride, flags, &base))) return rc;
  const size_t first = mlora_workspace_bytes(route->tokens, lora->rank_cap);  // a multiple of 256
  const size_t part = partials_of(w, route, base, flags);  // of the kernels this launch (its x_stride) runs
  if (first > MLORA_NOALLOC_SCRATCH_BYTES || part > MLORA_NOALLOC_SCRATCH_BYTES - first) return MLORA_EWORKSPACE;
  uint8_t* sp = noalloc_scratch();
  if (sp == nullptr) return MLORA_ELAUNCH;
  return mlora_int4_linear(w, lora, route, x, x_stride, y, y_stride, last_out, sp, first, part ? sp + first : nullptr,
                           part, flags, stream);
}

int mlora_int4_base_expand(const mlora_int4_t* w, const mlora_lora_t* lora, const mlora_route_t* route,
                           const uint16_t* x, int64_t x_stride, uint16_t* y, int64_t y_stride, uint16_t* last_out,
                           const uint16_t* mid, void* partials, size_t partials_bytes, int32_t flags, void* stream) {
  int rc = check_int4(w);
  if (rc) return rc;
  if ((rc = check_route(route)) || (rc = check_lora(lora, w->k, w->out)) || (rc = check_first_factors(route, lora)))
    return rc;
  if (route->tokens == 0) return MLORA_OK;
  if ((rc = check_rows(x, x_stride, w->k))) return rc;
  if (y == nullptr || y_stride < (gated_width(w, flags) ? w->out / 2 : w->out) || mid == nullptr || !aligned16(mid))
    return MLORA_EINVAL;
  Base base;
  if ((rc = base_of(w, lora, route, x_stride, flags, &base))) return rc;
  // mid is read only (fuse_shrink false)
  return run_base(w, lora, route, x, x_stride, y, y_stride, last_out, const_cast<uint16_t*>(mid), false, partials,
                  partials_bytes, base, flags, static_cast<hipStream_t>(stream));
}

int mlora_lora_add(const mlora_lora_t* lora, const mlora_route_t* route, const uint16_t* x, int64_t x_stride,
                   int32_t k, uint16_t* y, int64_t y_stride, int32_t n_out, void* workspace, size_t workspace_bytes,
                   int32_t flags, void* stream) {
  int rc = check_route(route);
  if (rc) return rc;
  if (k <= 0 || k % 64 || n_out <= 0) return MLORA_EINVAL;
  if ((rc = check_lora(lora, k, n_out)) || (rc = check_first_factors(route, lora))) return rc;
  if (route->tokens == 0) return MLORA_OK;
  if ((rc = check_rows(x, x_stride, k))) return rc;
  if (y == nullptr || y_stride < n_out) return MLORA_EINVAL;
  if (workspace == nullptr || !aligned16(workspace)) return MLORA_EWORKSPACE;
  if (workspace_bytes < mlora_workspace_bytes(route->tokens, lora->rank_cap)) return MLORA_EWORKSPACE;
  if (flags & (MLORA_FORCE_BASE_SPLIT | MLORA_EPILOGUE_SILU_MUL | MLORA_EPILOGUE_RESIDUAL))
    return MLORA_EUNSUPPORTED;  // y is updated in place
  const bool gemv = (flags & MLORA_FORCE_BASE_GEMV) || (!(flags & MLORA_FORCE_BASE_MFMA) && route->tokens <= 8);
  if (gemv && route->tokens > 8) return MLORA_EUNSUPPORTED;
  hipStream_t s = static_cast<hipStream_t>(stream);
  uint16_t* mid = static_cast<uint16_t*>(workspace);
  if ((rc = launch_shrink(*lora, *route, x, x_stride, k, mid, shrink_on_mfma(route, lora->pool_rows, flags), s)))
    return rc;
  return launch_base(nullptr, *lora, *route, x, x_stride, y, y_stride, nullptr, n_out, mid, gemv, s);
}

int mlora_readout_logits(const uint16_t* hidden, int64_t hidden_stride, int32_t dim, const uint16_t* readout_pool,
                         int64_t pool_stride, int32_t options, int32_t pool_rows, const int32_t* adapters,
                         int32_t rows, float* logits, void* stream) {
  if (rows < 0 || dim <= 0 || options <= 0 || pool_rows < 1) return MLORA_EINVAL;
  if (dim % 8 || dim > MLORA_READOUT_MAX_DIM || options > MLORA_READOUT_MAX_OPTIONS) return MLORA_EUNSUPPORTED;
  if (rows == 0) return MLORA_OK;
  if (hidden == nullptr || readout_pool == nullptr || adapters == nullptr || logits == nullptr) return MLORA_EINVAL;
  if (hidden_stride < dim || pool_stride < (int64_t)options * dim) return MLORA_EINVAL;
  if (!aligned16(hidden) || !aligned16(readout_pool) || hidden_stride % 8 || pool_stride % 8) return MLORA_EALIGN;
  return launch_readout_logits(hidden, hidden_stride, dim, readout_pool, pool_stride, options, pool_rows, adapters,
                               rows, logits, static_cast<hipStream_t>(stream));
}

int mlora_option_softmax(const float* logits, int32_t options, const int32_t* adapters, const int32_t* counts,
                         const float* temp_pool, int32_t pool_rows, int32_t rows, float* probs, void* stream) {
  if (rows < 0 || options <= 0 || pool_rows < 1) return MLORA_EINVAL;
  if (options > MLORA_READOUT_MAX_OPTIONS) return MLORA_EUNSUPPORTED;
  if (rows == 0) return MLORA_OK;
  if (logits == nullptr || adapters == nullptr || counts == nullptr || temp_pool == nullptr || probs == nullptr)
    return MLORA_EINVAL;
  return launch_option_softmax(logits, options, adapters, counts, temp_pool, pool_rows, rows, probs,
                               static_cast<hipStream_t>(stream));
}

int mlora_add_rms(const uint16_t* x, int64_t x_stride, const uint16_t* d, int64_t d_stride, const float* w1,
                  uint16_t* xo, int64_t xo_stride, uint16_t* h, int64_t h_stride, int64_t rows, int32_t n, float eps,
                  void* stream) {
  if (rows < 0 || n <= 0 || !(eps >= 0.0f)) return MLORA_EINVAL;
  if (n % 8 || n > MLORA_EPILOGUE_MAX_N) return MLORA_EUNSUPPORTED;
  if (rows == 0) return MLORA_OK;
  if (x == nullptr || w1 == nullptr || h == nullptr || (d != nullptr && xo == nullptr)) return MLORA_EINVAL;
  if (x_stride < n || h_stride < n || (d != nullptr && (d_stride < n || xo_stride < n))) return MLORA_EINVAL;
  if (!aligned16(x) || !aligned16(w1) || !aligned16(h) || x_stride % 8 || h_stride % 8) return MLORA_EALIGN;
  if (d != nullptr && (!aligned16(d) || !aligned16(xo) || d_stride % 8 || xo_stride % 8)) return MLORA_EALIGN;
  return launch_add_rms(x, x_stride, d, d_stride, w1, xo, xo_stride, h, h_stride, rows, n, eps,
                        static_cast<hipStream_t>(stream));
}

int mlora_silu_mul(const uint16_t* gu, int64_t gu_stride, uint16_t* y, int64_t y_stride, int64_t rows, int32_t inter,
                   void* stream) {
  if (rows < 0 || inter <= 0) return MLORA_EINVAL;
  if (inter % 8) return MLORA_EUNSUPPORTED;
  if (rows == 0) return MLORA_OK;
  if (gu == nullptr || y == nullptr || gu_stride < 2 * (int64_t)inter || y_stride < inter) return MLORA_EINVAL;
  if (!aligned16(gu) || !aligned16(y) || gu_stride % 8 || y_stride % 8) return MLORA_EALIGN;
  if (rows >= (((int64_t)1 << 31) * 256) / (inter / 8)) return MLORA_EOVERFLOW;  // rows * inter / 8 < 2^39
  return launch_silu_mul(gu, gu_stride, y, y_stride, rows, inter, static_cast<hipStream_t>(stream));
}

}  // extern "C"
#pragma GCC visibility pop
