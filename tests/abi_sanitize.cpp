// Host-side exercise of the C ABI's argument checks under AddressSanitizer and UndefinedBehaviorSanitizer (built and
// run by tests/test_abi_sanitized.py on a machine without a GPU). Every call below is one the library must refuse
// (or answer on the host) before any launch: null, misaligned, inconsistent and extreme arguments, sizes at the edge
// of the 32- and 64-bit index ranges. Prints each mismatch and exits 1 when there is one.
#include <cstdint>
#include <cstdio>

#include "jeff_mlora.h"

namespace {

int failures = 0;

void expect(const char* what, int got, int want) {
  if (got != want) {
    std::printf("MISMATCH %s: got %d, want %d\n", what, got, want);
    ++failures;
  }
}

// Addresses that are never dereferenced: the checks must stop before any use.
void* const A16 = reinterpret_cast<void*>(uintptr_t{1} << 20);
void* const A8 = reinterpret_cast<void*>((uintptr_t{1} << 20) + 8);

template <typename T>
T* p(void* v) {
  return static_cast<T*>(v);
}

mlora_lora_t lora_of(int32_t k, int32_t cols, int32_t cap) {
  mlora_lora_t L = {};
  L.pool = p<const uint16_t>(A16);
  L.ranks = p<const int32_t>(A16);
  L.off_a = 0;
  L.off_b[0] = (int64_t)cap * k;
  L.pool_stride = (int64_t)cap * k + (int64_t)cols * cap;
  L.ranks_stride = 1;
  L.pool_rows = 2;
  L.n_mats = 1;
  L.rank_cap = cap;
  L.cap[0] = cap;
  L.cols[0] = cols;
  return L;
}

mlora_route_t route_of(int64_t tokens, int32_t requests, int32_t max_segs) {
  int32_t* q = p<int32_t>(A16);
  return mlora_route_t{q, q, q, q, q, q, q, q, tokens, requests, max_segs};
}

}  // namespace

int main() {
  expect("abi version", mlora_abi_version(), MLORA_ABI_VERSION);
  expect("capture id without an output", mlora_capture_id(nullptr, nullptr), MLORA_EINVAL);
  expect("workspace bytes of nothing", (int)mlora_workspace_bytes(0, 16), 256);
  expect("workspace bytes, negative", (int)mlora_workspace_bytes(-5, -1), 256);

  // the kernel plan: host only, every extreme refused or answered without overflow
  int32_t b = 0, s = 0, r = 0;
  expect("plan null outputs", mlora_int4_plan(64, 64, 64, 8, 8, 9, 16, 0, nullptr, &s, &r), MLORA_EINVAL);
  expect("plan gemv", mlora_int4_plan(2048, 4096, 4096, 8, 8, 65, 192, 0, &b, &s, &r), MLORA_OK);
  expect("plan gemv base", b, 0);
  expect("plan narrow", mlora_int4_plan(2048, 4096, 4096, 256, 256, 65, 192, 0, &b, &s, &r), MLORA_OK);
  expect("plan narrow base", b, 3);
  expect("plan split", mlora_int4_plan(2048, 12288, 12288, 600, 600, 1025, 128, 0, &b, &s, &r), MLORA_OK);
  expect("plan split base", b, 2);
  expect("plan decode pool", mlora_int4_plan(2048, 12288, 12288, 4096, 4096, 1025, 128, 0, &b, &s, &r), MLORA_OK);
  expect("plan decode pool base", b, 1);
  expect("plan decode pool shrink", s, 0);
  expect("plan fused", mlora_int4_plan(1024, 3072, 3072, 8704, 64, 17, 16, 0, &b, &s, &r), MLORA_OK);
  expect("plan fused base", b, 1);
  expect("plan fused shrink", s, 1);
  expect("plan tokens at the int64 edge", mlora_int4_plan(64, 64, 64, INT64_MAX, 8, 9, 16, 0, &b, &s, &r),
         MLORA_EOVERFLOW);
  expect("plan inputs at the int32 edge", mlora_int4_plan(INT32_MAX - 63, 64, 64, 8, 8, 9, 16, 0, &b, &s, &r),
         MLORA_EOVERFLOW);
  expect("plan large inputs and columns",
         mlora_int4_plan((1 << 30), (1 << 30), (1 << 30), 1 << 20, 8, 9, 16, 0, &b, &s, &r), MLORA_EOVERFLOW);
  expect("plan forced gemv on many tokens",
         mlora_int4_plan(64, 64, 64, 9, 9, 10, 16, MLORA_FORCE_BASE_GEMV, &b, &s, &r), MLORA_EUNSUPPORTED);
  expect("plan ranges not dividing", mlora_int4_plan(192, 64, 64, 9, 9, 10, 16, MLORA_FORCE_BASE_NARROW |
         MLORA_FORCE_RANGES(2), &b, &s, &r), MLORA_EUNSUPPORTED);
  expect("plan ranges of 3", mlora_int4_plan(192, 64, 64, 9, 9, 10, 16, MLORA_FORCE_BASE_NARROW |
         MLORA_FORCE_RANGES(3), &b, &s, &r), MLORA_EUNSUPPORTED);
  expect("plan ranges of 15", mlora_int4_plan(1024, 64, 64, 9, 9, 10, 16, MLORA_FORCE_RANGES(15), &b, &s, &r),
         MLORA_EUNSUPPORTED);
  expect("plan negative requests", mlora_int4_plan(64, 64, 64, 8, -1, 9, 16, 0, &b, &s, &r), MLORA_EINVAL);

  // routing
  mlora_route_t rt = route_of(10, 10, 10);
  expect("route null adp", mlora_route(nullptr, nullptr, 1, &rt, 4, nullptr), MLORA_EINVAL);
  expect("route null route", mlora_route(p<int32_t>(A16), nullptr, 1, nullptr, 4, nullptr), MLORA_EINVAL);
  mlora_route_t many = route_of(10, MLORA_MAX_REQUESTS + 1, 1);
  expect("route too many requests", mlora_route(p<int32_t>(A16), nullptr, 1, &many, 4, nullptr),
         MLORA_EUNSUPPORTED);
  mlora_route_t few = route_of(10, 10, 1);
  expect("route too few segments", mlora_route(p<int32_t>(A16), nullptr, 1, &few, 4, nullptr), MLORA_EINVAL);
  expect("route rows of 2 are not 10 tokens", mlora_route(p<int32_t>(A16), nullptr, 2, &rt, 4, nullptr),
         MLORA_EINVAL);
  expect("route row_len overflowing", mlora_route(p<int32_t>(A16), nullptr, INT32_MAX, &rt, 4, nullptr),
         MLORA_EINVAL);
  mlora_route_t huge = route_of(INT64_MAX, 10, 10);
  expect("route tokens at the int64 edge", mlora_route(p<int32_t>(A16), nullptr, 1, &huge, 4, nullptr),
         MLORA_EOVERFLOW);
  expect("route pool rows 0", mlora_route(p<int32_t>(A16), nullptr, 1, &rt, 0, nullptr), MLORA_EINVAL);

  // dequantisation
  mlora_int4_t w = {p<const int32_t>(A16), p<const uint16_t>(A16), nullptr, 1024, 3072, 3072, 96};
  expect("dequant group 96", mlora_dequant(&w, p<uint16_t>(A16), nullptr), MLORA_EUNSUPPORTED);
  w.group = 64;
  w.k = 1000;
  expect("dequant k not a multiple of the group", mlora_dequant(&w, p<uint16_t>(A16), nullptr), MLORA_EINVAL);
  w.k = 1024;
  w.words = p<const int32_t>(A8);
  expect("dequant misaligned words", mlora_dequant(&w, p<uint16_t>(A16), nullptr), MLORA_EALIGN);
  w.words = p<const int32_t>(A16);
  expect("dequant misaligned output", mlora_dequant(&w, p<uint16_t>(A8), nullptr), MLORA_EALIGN);
  mlora_int4_t big = {p<const int32_t>(A16), p<const uint16_t>(A16), nullptr, 1 << 20, 1 << 14, 1 << 14, 64};
  expect("dequant words past 2^31", mlora_dequant(&big, p<uint16_t>(A16), nullptr), MLORA_EOVERFLOW);
  expect("dequant null", mlora_dequant(nullptr, nullptr, nullptr), MLORA_EINVAL);

  // products: argument errors before any launch
  mlora_int4_t w64 = {p<const int32_t>(A16), p<const uint16_t>(A16), nullptr, 64, 64, 64, 64};
  mlora_lora_t L = lora_of(64, 64, 64);
  mlora_route_t r1 = route_of(1 << 24, 1, 1);  // first factors of exactly 2^31 bytes
  expect("linear first factors at 2^31", mlora_int4_linear(&w64, &L, &r1, p<uint16_t>(A16), 64, nullptr, 64, nullptr,
         A16, (size_t)1 << 40, nullptr, 0, 0, nullptr), MLORA_EOVERFLOW);
  mlora_route_t r2 = route_of((1 << 24) - 1, 1, 1);
  expect("linear without y", mlora_int4_linear(&w64, &L, &r2, p<uint16_t>(A16), 64, nullptr, 64, nullptr, A16,
         (size_t)1 << 40, nullptr, 0, 0, nullptr), MLORA_EINVAL);
  expect("linear misaligned x", mlora_int4_linear(&w64, &L, &r2, p<uint16_t>(A8), 64, p<uint16_t>(A16), 64, nullptr,
         A16, (size_t)1 << 40, nullptr, 0, 0, nullptr), MLORA_EALIGN);
  expect("linear small workspace", mlora_int4_linear(&w64, &L, &r2, p<uint16_t>(A16), 64, p<uint16_t>(A16), 64,
         nullptr, A16, 100, nullptr, 0, 0, nullptr), MLORA_EWORKSPACE);
  mlora_lora_t Lbad = L;
  Lbad.rank_cap = 48;
  expect("linear caps not summing to the rank", mlora_int4_linear(&w64, &Lbad, &r2, p<uint16_t>(A16), 64,
         p<uint16_t>(A16), 64, nullptr, A16, (size_t)1 << 40, nullptr, 0, 0, nullptr), MLORA_EINVAL);
  Lbad = L;
  Lbad.off_b[0] = INT64_MAX - 7;
  expect("linear sB offset at the int64 edge", mlora_int4_linear(&w64, &Lbad, &r2, p<uint16_t>(A16), 64,
         p<uint16_t>(A16), 64, nullptr, A16, (size_t)1 << 40, nullptr, 0, 0, nullptr), MLORA_EINVAL);
  Lbad = L;
  Lbad.cols[0] = INT32_MAX;
  Lbad.cap[0] = INT32_MAX - 7;
  expect("linear columns times capacity near int64", mlora_int4_linear(&w64, &Lbad, &r2, p<uint16_t>(A16), 64,
         p<uint16_t>(A16), 64, nullptr, A16, (size_t)1 << 40, nullptr, 0, 0, nullptr), MLORA_EINVAL);
  Lbad = L;
  Lbad.n_mats = MLORA_MAX_MATS + 1;
  expect("linear too many matrices", mlora_int4_linear(&w64, &Lbad, &r2, p<uint16_t>(A16), 64, p<uint16_t>(A16), 64,
         nullptr, A16, (size_t)1 << 40, nullptr, 0, 0, nullptr), MLORA_EUNSUPPORTED);
  mlora_route_t r0 = route_of(0, 0, 0);
  expect("linear of no tokens", mlora_int4_linear(&w64, &L, &r0, nullptr, 0, nullptr, 0, nullptr, nullptr, 0, nullptr,
         0, 0, nullptr), MLORA_OK);
  expect("linear null descriptors", mlora_int4_linear(nullptr, nullptr, nullptr, nullptr, 0, nullptr, 0, nullptr,
         nullptr, 0, nullptr, 0, 0, nullptr), MLORA_EINVAL);
  expect("no-alloc first factors at 2^31", mlora_int4_linear_noalloc(&w64, &L, &r1, p<uint16_t>(A16), 64, nullptr,
         64, nullptr, 0, nullptr), MLORA_EOVERFLOW);
  expect("no-alloc of no tokens", mlora_int4_linear_noalloc(&w64, &L, &r0, nullptr, 0, nullptr, 0, nullptr, 0,
         nullptr), MLORA_OK);
  expect("no-alloc null descriptors", mlora_int4_linear_noalloc(nullptr, nullptr, nullptr, nullptr, 0, nullptr, 0,
         nullptr, 0, nullptr), MLORA_EINVAL);
  mlora_int4_t w12 = {p<const int32_t>(A16), p<const uint16_t>(A16), nullptr, 2048, 12288, 12288, 128};
  mlora_lora_t L12 = lora_of(2048, 12288, 16);
  mlora_route_t r4096 = route_of(4096, 4096, 2);
  expect("no-alloc partials beyond the scratch", mlora_int4_linear_noalloc(&w12, &L12, &r4096, p<uint16_t>(A16),
         2048, p<uint16_t>(A16), 12288, nullptr, MLORA_FORCE_BASE_SPLIT | MLORA_FORCE_SHRINK_SEGMENT, nullptr),
         MLORA_EWORKSPACE);
  expect("no-alloc x stride at the int64 edge", mlora_int4_linear_noalloc(&w12, &L12, &r4096, p<uint16_t>(A16),
         INT64_MAX / 16 * 8, p<uint16_t>(A16), 12288, nullptr, MLORA_FORCE_BASE_SPLIT, nullptr), MLORA_EUNSUPPORTED);
  mlora_lora_t Lwide = L;
  Lwide.pool_stride = INT64_MAX - 7;
  Lwide.off_a = 8;
  expect("pool stride at the int64 edge", mlora_int4_linear(&w64, &Lwide, &r2, p<uint16_t>(A16), 64, nullptr, 64,
         nullptr, A16, (size_t)1 << 40, nullptr, 0, 0, nullptr), MLORA_EINVAL);
  expect("partials of a forced split", mlora_int4_partials_bytes(&w12, &L12, &r4096, MLORA_FORCE_BASE_SPLIT) >
         MLORA_NOALLOC_SCRATCH_BYTES, 1);
  expect("partials of null", (int)mlora_int4_partials_bytes(nullptr, nullptr, nullptr, 0), 0);
  expect("base_expand without mid", mlora_int4_base_expand(&w64, &L, &r2, p<uint16_t>(A16), 64, p<uint16_t>(A16), 64,
         nullptr, nullptr, nullptr, 0, 0, nullptr), MLORA_EINVAL);
  expect("shrink first factors at 2^31", mlora_shrink(&L, &r1, p<uint16_t>(A16), 64, 64, p<uint16_t>(A16), 0,
         nullptr), MLORA_EOVERFLOW);
  expect("shrink k not a multiple of 64", mlora_shrink(&L, &r2, p<uint16_t>(A16), 64, 96, p<uint16_t>(A16), 0,
         nullptr), MLORA_EINVAL);
  expect("lora_add forced split", mlora_lora_add(&L, &r2, p<uint16_t>(A16), 64, 64, p<uint16_t>(A16), 64, 64, A16,
         (size_t)1 << 40, MLORA_FORCE_BASE_SPLIT, nullptr), MLORA_EUNSUPPORTED);
  expect("lora_add first factors at 2^31", mlora_lora_add(&L, &r1, p<uint16_t>(A16), 64, 64, p<uint16_t>(A16), 64, 64,
         A16, (size_t)1 << 40, 0, nullptr), MLORA_EOVERFLOW);

  // the decision head and the element-wise steps
  expect("readout dim not a multiple of 8", mlora_readout_logits(p<uint16_t>(A16), 20, 20, p<uint16_t>(A16), 4000,
         200, 4, p<int32_t>(A16), 8, p<float>(A16), nullptr), MLORA_EUNSUPPORTED);
  expect("readout too many options", mlora_readout_logits(p<uint16_t>(A16), 64, 64, p<uint16_t>(A16), 1 << 20, 257, 4,
         p<int32_t>(A16), 8, p<float>(A16), nullptr), MLORA_EUNSUPPORTED);
  expect("readout pool stride too small", mlora_readout_logits(p<uint16_t>(A16), 64, 64, p<uint16_t>(A16), 64, 200, 4,
         p<int32_t>(A16), 8, p<float>(A16), nullptr), MLORA_EINVAL);
  expect("softmax no options", mlora_option_softmax(p<float>(A16), 0, p<int32_t>(A16), p<int32_t>(A16),
         p<float>(A16), 4, 8, p<float>(A16), nullptr), MLORA_EINVAL);
  expect("add_rms negative eps", mlora_add_rms(p<uint16_t>(A16), 64, nullptr, 0, p<float>(A16), nullptr, 0,
         p<uint16_t>(A16), 64, 4, 64, -1.0f, nullptr), MLORA_EINVAL);
  expect("add_rms misaligned weight", mlora_add_rms(p<uint16_t>(A16), 64, nullptr, 0, p<float>(A8), nullptr, 0,
         p<uint16_t>(A16), 64, 4, 64, 1e-6f, nullptr), MLORA_EALIGN);
  expect("add_rms rows too long", mlora_add_rms(p<uint16_t>(A16), 1 << 20, nullptr, 0, p<float>(A16), nullptr, 0,
         p<uint16_t>(A16), 1 << 20, 4, MLORA_EPILOGUE_MAX_N + 8, 1e-6f, nullptr), MLORA_EUNSUPPORTED);
  expect("silu_mul rows past the index range", mlora_silu_mul(p<uint16_t>(A16), 1 << 14, p<uint16_t>(A16), 1 << 13,
         INT64_MAX / 2, 1 << 13, nullptr), MLORA_EOVERFLOW);
  expect("silu_mul stride too small", mlora_silu_mul(p<uint16_t>(A16), 64, p<uint16_t>(A16), 64, 4, 64, nullptr),
         MLORA_EINVAL);

  std::printf("%s: %d mismatches\n", failures ? "FAILED" : "ok", failures);
  return failures ? 1 : 0;
}
