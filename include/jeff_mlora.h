/* jeff_mlora.h: C ABI of the MI355X (gfx950) batched multi-LoRA INT4 linear.
 *
 * One fused group of matrices that read the same input x (T tokens, K inputs) and are stacked along the output:
 *   y[t, :] = bf16( x[t] W^T  +  bf16(x[t] A_j^T) (sB_j)^T  for each matrix j of the group )
 * with W = bf16((c - z) s) from packed 4-bit codes, and (A_j, sB_j) read from the pool row of token t's adapter.
 * Every entry point takes raw device pointers, sizes and a HIP stream, allocates no memory, never synchronises, and
 * returns MLORA_OK or a negative status before launching anything. No C++ exception crosses this boundary.
 * A narrow product (at most 256 tokens, few per adapter segment: decode) is two launches on the caller's stream, the
 * first factor then the base product with the second factor fused, plus a third that adds the float32 ranges when
 * the input dimension is split. A split product (more tokens, few per segment) is three: the first factor, the base
 * ranges, then the epilogue. Every launch of every entry point goes to the stream passed in; the library keeps no
 * streams, events or device buffers of its own, so calls from several host threads on several streams are safe as
 * long as they do not share route, workspace, partials or output buffers (calls that share them race, as any two
 * kernels writing one buffer do).
 *
 * Reference interfaces replaced (paths in the reference checkout, runtime/python/src/jeff_runtime/engine/):
 *   mlora_route        per-token adapter lookup adp[t // row_len]          fast_path.py:167,189; int4_kernels.py:72,113
 *   mlora_int4_linear  int4_product (base + LoRA shrink + expand)          int4_kernels.py:132-177
 *   mlora_lora_add     lora_add (in-place LoRA update of y)                fast_path.py:277-289
 *   mlora_shrink       the LoRA first factor QP = x A^T (_lora_mid_kernel) fast_path.py:159-177
 *   mlora_int4_base_expand  the base tiles + LoRA output epilogue          int4_kernels.py:44-64,105-129
 *   mlora_dequant      dequantize / bf16(q * s) of the kernel layout       int4.py:203-208,258-262
 *   mlora_int4_plan    int4_tiles (the tile and kernel choice of a shape)   int4_tiles.py:57-71
 *   mlora_workspace_bytes  Workspace.QP sizing                             fast_path.py:261-274
 *   mlora_int4_partials_bytes  Workspace.P sizing (split partial products)  int4_kernels.py:150-166
 *   mlora_int4_partials_bound  Workspace sizing from its shapes up front     fast_path.py:261-274
 *   mlora_readout_logits  readout_logits (per-adapter readout)          batched_kernels.py:492-504,522-536
 *   mlora_option_softmax  option_softmax (mask, temperature, softmax)     batched_kernels.py:507-519,539-553
 *   mlora_add_rms      add_rms / rms (residual add + RMSNorm)              fast_path.py:80-100,295-298
 *   mlora_silu_mul     silu_mul (SiLU of the gate half times the up half)  fast_path.py:141-156
 *   mlora_capture_id   no counterpart: the reference's kernels read adp themselves in every product
 *                      (fast_path.py:167,189), so it needs no separate routing launch to share between them; the
 *                      Python Workspace uses this to decide whether a route launched earlier in the same graph
 *                      capture can be shared (jeff_amd/fast_path.py Workspace.routed)
 */
#ifndef JEFF_MLORA_H
#define JEFF_MLORA_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MLORA_ABI_VERSION 2
#define MLORA_MAX_MATS 8            /* matrices per fused group (the reference's largest has 4) */
#define MLORA_MAX_REQUESTS 8192     /* request rows per routed pass */
#define MLORA_MAX_POOL_ROWS 262144  /* adapter pool rows (row 0 = the base, no update) */
#define MLORA_READOUT_MAX_DIM 2048  /* hidden size of the decision head's readout */
#define MLORA_READOUT_MAX_OPTIONS 256  /* answer options per readout */
#define MLORA_EPILOGUE_MAX_N 8192   /* row length of add_rms */
#define MLORA_NOALLOC_SCRATCH_BYTES (64u << 20)  /* device scratch of mlora_int4_linear_noalloc, per GPU */

enum {
  MLORA_OK = 0,
  MLORA_EINVAL = -1,       /* a null pointer, a bad size or shape */
  MLORA_EALIGN = -2,       /* a pointer, stride or offset not 16-byte aligned */
  MLORA_EOVERFLOW = -3,    /* sizes beyond the kernels' index range */
  MLORA_EWORKSPACE = -4,   /* workspace too small */
  MLORA_EUNSUPPORTED = -5, /* a shape this build does not run (group, matrices, requests) */
  MLORA_ELAUNCH = -6       /* the HIP launch itself failed */
};

/* Route status bits, written by mlora_route to route->status[0] on the device. */
#define MLORA_ROUTE_BAD_ADAPTER 1   /* an adapter index outside [0, pool_rows): that row was routed to row 0 */
#define MLORA_ROUTE_BAD_SEQLENS 2   /* cu_seqlens not 0-based, non-decreasing, ending at tokens: identity routing */

/* Kernel-selection flags (0 = automatic). */
#define MLORA_FORCE_BASE_GEMV 1
#define MLORA_FORCE_BASE_MFMA 2
#define MLORA_FORCE_SHRINK_SEGMENT 4
#define MLORA_FORCE_SHRINK_MFMA 8
#define MLORA_FORCE_BASE_SPLIT 16   /* split product: float32 partials, then a per-segment epilogue launch */
#define MLORA_FORCE_BASE_NARROW 32  /* narrow product (at most 256 tokens): every token in one row tile of 64 columns */
#define MLORA_FORCE_RANGES(s) ((s) << 8)  /* a narrow product over s = 1, 2, 4 or 8 input ranges (s dividing k / 64) */
/* Epilogue flag: the group is a gate_up pair (matrix 0 gate, matrix 1 up, out / 2 columns each, out a multiple of
 * 256, one rank capacity of at most 64 for both); y (and last_out) receive silu(gate) * up, out / 2 columns per row,
 * each element
 * bf16(bf16(g / (1 + exp(-g))) * u) of the product's rounded gate and up outputs, the bits mlora_silu_mul gives on
 * the unfused product. Products with this flag never take the GEMV kernel; the split product needs capacities in
 * {0, 8, 16, 32, 64}; mlora_lora_add refuses it. */
#define MLORA_EPILOGUE_SILU_MUL 64
/* Epilogue flag: the residual add of add_rms (fast_path.py:80-100, x = bf16(x + d)) in the product's output tile. y
 * holds the residual rows on entry (row t at y + t * y_stride) and receives bf16(residual + output) with the output
 * rounded to bf16 first, the bits mlora_add_rms writes for x + d on the unfused product; last_out (when given)
 * receives the same sums. y must not overlap x. Not with MLORA_EPILOGUE_SILU_MUL (MLORA_EINVAL); products with this
 * flag never take the GEMV kernel; the fused product needs tokens * max(x_stride, k) below 2^31 and the split product
 * capacities in {0, 8, 16, 32, 64} (MLORA_EUNSUPPORTED otherwise); mlora_lora_add refuses it. */
#define MLORA_EPILOGUE_RESIDUAL 128

/* INT4 weights in the kernel layout (reference int4.py:215-230, plus zero points and g128):
 * words  int32 (k/8, columns): word i of column c holds inputs 8i..8i+7, input 8i+j in bits 4j..4j+3 (the code c);
 * scales bf16 (k/group, columns); zeros uint8 (k/group, columns) with z in [0, 15], or NULL for z = 8 (symmetric);
 * columns = out rounded up to 64; padding columns hold code 8, zero 8, scale 1. */
typedef struct {
  const int32_t* words;
  const uint16_t* scales;
  const uint8_t* zeros;
  int32_t k, columns, out, group;
} mlora_int4_t;

/* The adapter pool of one fused group. Row a of the pool (pool + a * pool_stride, bf16) holds, for this group:
 * at off_a the stacked first factors A (rank_cap, k): matrix j in rows [rho_j, rho_j + cap[j]), rho_j = sum of the
 * caps before j; at off_b[j] the second factor of matrix j, sB_j (cols[j], s), row n = output n's rank vector, in a
 * block of cols[j] * cap[j] elements. The row stride s depends on the row's live rank r of matrix j:
 * s = mlora_sb_stride(r, cap[j]) (r rounded up to a power of two, at least 8, at most cap[j]), so a low-rank adapter's
 * sB is dense. ranks[a * ranks_stride + j] is the live rank of matrix j in row a (0: no update); only rows [0, r) of
 * A_j and columns [0, r) of sB_j are read. Row 0 is the base and must have all ranks 0. */
static inline int32_t mlora_sb_stride(int32_t rank, int32_t cap) {
  int32_t s = 8;
  while (s < rank) s <<= 1;
  return s < cap ? s : cap;
}
typedef struct {
  const uint16_t* pool;
  const int32_t* ranks;
  int64_t pool_stride;
  int64_t off_a;
  int64_t off_b[MLORA_MAX_MATS];
  int32_t ranks_stride, pool_rows, n_mats, rank_cap;
  int32_t cap[MLORA_MAX_MATS];
  int32_t cols[MLORA_MAX_MATS];
} mlora_lora_t;

/* A routed pass: request rows sorted (stably) by adapter index, so each adapter's tokens form one segment.
 * Buffers on the device, written by mlora_route and read by the products:
 *   req_order (requests)        request rows in sorted order
 *   tok_perm  (tokens)          sorted token position -> original token index
 *   last_of   (tokens)          per sorted position, the request whose last token is there, else -1
 *   seg_of    (tokens)          per sorted position, the segment it belongs to
 *   seg_start (max_segs + 1)    first sorted position of each segment, then the end
 *   seg_adapter (max_segs)      the pool row of each segment, increasing
 *   num_segs, status (1 each)   the number of segments; MLORA_ROUTE_* bits
 * max_segs must be at least min(requests, pool_rows). */
typedef struct {
  int32_t* req_order;
  int32_t* tok_perm;
  int32_t* last_of;
  int32_t* seg_of;
  int32_t* seg_start;
  int32_t* seg_adapter;
  int32_t* num_segs;
  int32_t* status;
  int64_t tokens;
  int32_t requests, max_segs;
} mlora_route_t;

int mlora_abi_version(void);

/* *id = the HIP capture sequence id of `stream` while it is capturing a graph, else 0. MLORA_ELAUNCH when HIP
 * cannot say (e.g. the legacy stream queried during another stream's global-mode capture). */
int mlora_capture_id(void* stream, uint64_t* id);

/* Bytes of device workspace a product over `tokens` tokens of a group with `rank_cap` stacked ranks needs. */
size_t mlora_workspace_bytes(int64_t tokens, int32_t rank_cap);

/* Route a pass: adp int32 (requests) pool rows; either cu_seqlens int32 (requests + 1) token offsets or, when it
 * is NULL, rows of row_len tokens each (tokens = requests * row_len). One launch. */
int mlora_route(const int32_t* adp, const int32_t* cu_seqlens, int32_t row_len, const mlora_route_t* route,
                int32_t pool_rows, void* stream);

/* The kernels mlora_int4_linear runs, without running them (host only, no GPU needed): for a pass of `tokens` tokens
 * in `requests` request rows over a pool of pool_rows rows, through a group of k inputs, `columns` kernel columns,
 * `out` outputs and rank_cap stacked ranks, with these flags. *base: 0 the GEMV (at most 8 tokens), 1 the MFMA tile
 * kernel with the second factor fused, 2 the split product, 3 the narrow product; *shrink: 0 the segment form, 1
 * the MFMA form of the first factor; *ranges: input ranges of a split or narrow product (1 otherwise; the narrow
 * count depends on the current device's CU count, 256 without a device). MLORA_EUNSUPPORTED as mlora_int4_linear
 * would return it for forced flags that cannot run. */
int mlora_int4_plan(int32_t k, int32_t columns, int32_t out, int64_t tokens, int32_t requests, int32_t pool_rows,
                    int32_t rank_cap, int32_t flags, int32_t* base, int32_t* shrink, int32_t* ranges);

/* The dequantised weights bf16((c - z) s) of `w` as bf16 (out, k), row-major. */
int mlora_dequant(const mlora_int4_t* w, uint16_t* out, void* stream);

/* The LoRA first factor of every routed token: mid (tokens, rank_cap) bf16 at sorted positions, matrix j's live
 * ranks in columns [rho_j, rho_j + rank); other columns are not written. */
int mlora_shrink(const mlora_lora_t* lora, const mlora_route_t* route, const uint16_t* x, int64_t x_stride,
                 int32_t k, uint16_t* mid, int32_t flags, void* stream);

/* Bytes of float32 partial products the product of `w` over `route` needs with these flags; 0 when it runs the
 * fused kernels. Passes with few tokens per adapter segment (decode) split the input dimension into ranges whose
 * float32 sums a later launch adds in order (the reference's split product); its size depends on the token count,
 * the group's columns and inputs and the device's CU count, not on device memory, so a caller can size its buffer
 * once per shape. */
size_t mlora_int4_partials_bytes(const mlora_int4_t* w, const mlora_lora_t* lora, const mlora_route_t* route,
                                 int32_t flags);

/* y (tokens, w->out) bf16 = x W^T + each token's LoRA update, one rounding per output; x (tokens, k) bf16 rows
 * x_stride elements apart (k a multiple of 64, rows 16-byte aligned). last_out (requests, w->out) bf16 or NULL:
 * each request's last-token output row as well. workspace: the first factors (mlora_workspace_bytes);
 * partials: mlora_int4_partials_bytes of float32 scratch (NULL when that is 0). */
/* The most float32 partial bytes any product of a group of k inputs, `columns` kernel columns and `out` outputs over
 * at most `tokens` tokens needs under the automatic kernel choice (any request count, pool, epilogue or x stride),
 * so a workspace can be sized once from its shapes, before any pass is recorded (host only, no GPU needed; the
 * narrow range count follows the current device's CU count, 256 without a device). 0 for arguments no product
 * accepts. Forced kernel flags (tests) can need more: mlora_int4_partials_bytes says how much. */
size_t mlora_int4_partials_bound(int32_t k, int32_t columns, int32_t out, int64_t tokens);

int mlora_int4_linear(const mlora_int4_t* w, const mlora_lora_t* lora, const mlora_route_t* route,
                      const uint16_t* x, int64_t x_stride, uint16_t* y, int64_t y_stride, uint16_t* last_out,
                      void* workspace, size_t workspace_bytes, void* partials, size_t partials_bytes, int32_t flags,
                      void* stream);

/* mlora_int4_linear with its scratch inside the library: no counterpart in the reference, for callers that cannot
 * allocate device memory or pass a workspace (code under graph capture that must not allocate, tight serving loops,
 * harnesses that forbid hipMalloc). The first factors and any float32 partials live in a static device array of
 * MLORA_NOALLOC_SCRATCH_BYTES in the library's code object: every GPU on which the library's kernels are loaded
 * holds its own copy from then until the process ends, whether or not this entry point is called. The call
 * allocates nothing and returns MLORA_EWORKSPACE before any launch when a pass needs more (mlora_workspace_bytes
 * plus the partials of the kernels chosen for this call's x_stride). Every call on one GPU shares that GPU's array and leaves its contents behind; the
 * kernels write every scratch byte they read, so nothing needs clearing, but calls that overlap on one GPU (other
 * streams, other threads) race on it. Same arguments, results and bits as mlora_int4_linear otherwise. */
int mlora_int4_linear_noalloc(const mlora_int4_t* w, const mlora_lora_t* lora, const mlora_route_t* route,
                              const uint16_t* x, int64_t x_stride, uint16_t* y, int64_t y_stride, uint16_t* last_out,
                              int32_t flags, void* stream);

/* mlora_int4_linear without its shrink launch: the base product and the LoRA second factor, reading the first
 * factors mid (tokens, rank_cap) that mlora_shrink wrote for the same route and x. */
int mlora_int4_base_expand(const mlora_int4_t* w, const mlora_lora_t* lora, const mlora_route_t* route,
                           const uint16_t* x, int64_t x_stride, uint16_t* y, int64_t y_stride, uint16_t* last_out,
                           const uint16_t* mid, void* partials, size_t partials_bytes, int32_t flags, void* stream);

/* In place: y (tokens, n_out) bf16 += each token's LoRA update (y read in float32, one rounding); x (tokens, k). */
int mlora_lora_add(const mlora_lora_t* lora, const mlora_route_t* route, const uint16_t* x, int64_t x_stride,
                   int32_t k, uint16_t* y, int64_t y_stride, int32_t n_out, void* workspace, size_t workspace_bytes,
                   int32_t flags, void* stream);

/* The decision head's logits (the reference's readout_logits): for each of `rows` request rows, logits (rows,
 * options) float32 = bf16(sum_d readout_pool[adapters[b]][o][d] * hidden[b][d]) summed in float32. hidden bf16 (rows,
 * dim) rows hidden_stride apart; readout_pool bf16 (pool_rows, options, dim), adapters pool_stride elements apart;
 * adapters int32 (rows), an index outside [0, pool_rows) reads row 0. dim a multiple of 8, at most
 * MLORA_READOUT_MAX_DIM; options at most MLORA_READOUT_MAX_OPTIONS. */
int mlora_readout_logits(const uint16_t* hidden, int64_t hidden_stride, int32_t dim, const uint16_t* readout_pool,
                         int64_t pool_stride, int32_t options, int32_t pool_rows, const int32_t* adapters,
                         int32_t rows, float* logits, void* stream);

/* The decision head's probabilities (the reference's option_softmax): probs (rows, options) float32 = softmax over o
 * of (o < counts[b] ? logits[b][o] : -1e9) / temp_pool[adapters[b]]; temp_pool float32 (pool_rows). */
int mlora_option_softmax(const float* logits, int32_t options, const int32_t* adapters, const int32_t* counts,
                         const float* temp_pool, int32_t pool_rows, int32_t rows, float* probs, void* stream);

/* Residual add and RMSNorm of each of `rows` rows of n bf16 values (the reference's add_rms, and rms when d is NULL):
 * x' = bf16(x + d) (written to xo when d is given; xo may be x), h = bf16(x' * rsqrt(sum(x'^2) / n + eps) * w1), the
 * sum of squares in float32 in a fixed order. w1 float32 (n) = 1 + the norm's weight. n a multiple of 8, at most
 * MLORA_EPILOGUE_MAX_N; rows, w1 16-byte aligned, strides multiples of 8 elements. */
int mlora_add_rms(const uint16_t* x, int64_t x_stride, const uint16_t* d, int64_t d_stride, const float* w1,
                  uint16_t* xo, int64_t xo_stride, uint16_t* h, int64_t h_stride, int64_t rows, int32_t n, float eps,
                  void* stream);

/* The gated activation after the gate_up product (the reference's silu_mul): for each of `rows` rows of gu (the
 * gate half in columns 0..inter-1, the up half in inter..2 inter-1), y = bf16(bf16(g / (1 + exp(-g))) * u), the
 * quotient correctly rounded to float32 (signed zeros, infinities and NaN as the float32 formula gives them). inter
 * a multiple of 8; rows 16-byte aligned, strides multiples of 8 elements. */
int mlora_silu_mul(const uint16_t* gu, int64_t gu_stride, uint16_t* y, int64_t y_stride, int64_t rows, int32_t inter,
                   void* stream);

#ifdef __cplusplus
}
#endif

#endif /* JEFF_MLORA_H */
