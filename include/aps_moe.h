/*
 * aps_moe.h -- C ABI of the MI355X (gfx950) MoE feed-forward engine.
 *
 * Plain C: integer/pointer/size arguments only.  Every `void* stream` is a
 * hipStream_t (NULL = the legacy default stream, which is the ordering the
 * reference relies on: all of its kernels go to stream 0).  Every device
 * array is caller-owned device memory; every entry point except the weight
 * registration is asynchronous on `stream` and allocates nothing.
 *
 * Return codes: APS_OK (0) or a negative aps_status; aps_moe_last_error()
 * then gives a thread-local message.  The reference raises
 * std::invalid_argument / std::runtime_error for the same conditions
 * (src/tensor.cu:370-374, 2761-2764, 2793-2797); the C++ layer in
 * include/tensor.h turns these codes back into those exception types.
 *
 * Routing semantics are the reference's, bit for bit:
 *   logits[t][e] = fp32 FMA chain over k = 0..H-1 ascending, +0 init
 *   q = sign(l) * floorf(|l| / 1e-3f + 0.5f) * 1e-3f
 *   top-2 = greedy scan, later expert wins only if q > q_best + 2e-2f
 *   weights 0.5 / 0.5; stable counting sort by expert, ties by token.
 */
#ifndef APS_MOE_H
#define APS_MOE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define APS_MOE_ABI_VERSION 2  /* 2: aps_moe_ws_layout grew the slot-ordered lists */

#if defined(__GNUC__) || defined(__clang__)
#define APS_API __attribute__((visibility("default")))
#else
#define APS_API
#endif

typedef enum aps_status {
    APS_OK = 0,
    APS_ERR_SHAPE = -1,     /* inconsistent or unsupported sizes          */
    APS_ERR_HANDLE = -2,    /* weight handle 0, released or out of range   */
    APS_ERR_DTYPE = -3,     /* dtype code not supported for this argument  */
    APS_ERR_HIP = -4,       /* a HIP runtime call failed                   */
    APS_ERR_ARG = -5,       /* NULL pointer or other invalid argument      */
    APS_ERR_WORKSPACE = -6  /* workspace missing or smaller than required  */
} aps_status;

typedef enum aps_dtype {
    APS_DTYPE_F32 = 0,
    APS_DTYPE_BF16 = 1,
    APS_DTYPE_E4M3 = 2      /* OCP fp8 e4m3 ("fn"): bias 7, max 448        */
} aps_dtype;

/* Weight set of one MoE layer (the reference's MoeWeightSet,
 * src/tensor.cu:1216-1220).  w1/w3/w2 are HOST arrays of num_experts DEVICE
 * pointers in the reference's nn.Linear layout: w1[e], w3[e] are
 * [ffn][hidden], w2[e] is [hidden][ffn], row-major.
 * compute_dtype picks the kernels:
 *   APS_DTYPE_F32  - fp32 FMA-chain kernels, accumulation order identical to
 *                    the reference (k ascending), src_dtype must be F32;
 *   APS_DTYPE_BF16 - bf16 MFMA kernels, fp32 accumulate; src F32 or BF16;
 *   APS_DTYPE_E4M3 - fp8 MFMA kernels (config C5); src E4M3 codes
 *                    with per-output-channel fp32 scales (w1_scale[e],
 *                    w3_scale[e]: [ffn] device arrays, w2_scale[e]:
 *                    [hidden]); x (bf16) and the SwiGLU activations are
 *                    quantised per row at run time, scale = amax / 448,
 *                    round to nearest even; fused entry points only.
 * Registration copies the weights into the library's own packed layout
 * (the caller's buffers may be freed afterwards). */
typedef struct aps_moe_weights_desc {
    int32_t num_experts;
    int32_t hidden;
    int32_t ffn;
    int32_t src_dtype;
    int32_t compute_dtype;
    const void* const* w1;
    const void* const* w3;
    const void* const* w2;
    const float* const* w1_scale;
    const float* const* w3_scale;
    const float* const* w2_scale;
} aps_moe_weights_desc;

/* Byte offsets of the intermediate arrays inside a forward workspace, for
 * callers (and tests) that want to read the routing plan back. */
typedef struct aps_moe_ws_layout {
    size_t total_bytes;
    size_t logits;          /* f32 [rows][E]                        */
    size_t routes;          /* u8  [rows][2], slot 0 = first pick   */
    size_t tile_counts;     /* u32 [ceil(rows/64)][E]: byte q counts the
                               routes of tokens 16q..16q+15 of a tile */
    size_t counts;          /* u32 [E]                              */
    size_t offsets;         /* u32 [E+1]                            */
    size_t assignment_rows; /* u32 [2*rows] position -> token       */
    size_t route_positions; /* u32 [2*rows] (token, slot) -> position */
    size_t act;             /* [2*rows][ffn], f32 (F32 path) or bf16 */
    size_t act_scale;       /* fp8 path: f32 [2*rows] per-position scale */
    size_t y;               /* [2*rows][hidden], f32 (F32 path) or bf16 */
    size_t xq;              /* x in the compute dtype when the caller
                               passes another one: bf16 [rows][hidden]
                               (bf16 weights, fp32 x; it shares y's
                               bytes: dead before y is written), e4m3
                               (fp8 path, its own bytes) */
    size_t xq_scale;        /* fp8 path: f32 [rows] per-token scale */
    size_t actq;            /* fp8 path: e4m3 act [2*rows][ffn rounded
                               up to 128], zero padded              */
    size_t tile_counts0;    /* u32 [ceil(rows/64)][E]: as tile_counts,
                               slot-0 routes only (aps_moe_forward) */
    size_t slot1;           /* u32 [E]: offsets[e] + slot-0 routes of e */
    size_t slot_rows;       /* u32 [2*rows] slot-ordered list: entries
                               [offsets[e], slot1[e]) the positions of
                               e's slot-0 routes, [slot1[e], offsets[e+1])
                               of its slot-1 routes, tokens ascending  */
    size_t slot_tokens;     /* u32 [2*rows] the token of each entry  */
} aps_moe_ws_layout;

/* ---- weights ----------------------------------------------------------- */

/* Replaces tensor_ops::register_moe_weights_gpu (reference
 * include/tensor.h:142-145, src/tensor.cu:2757-2788).  Writes a 1-based
 * handle (0 is never a valid handle, as in the reference).  Synchronous.
 * num_experts 1..64; a one-expert set is a dense FFN for aps_mlp_forward
 * (the reference's PhiMLP weights), routing needs two or more. */
APS_API int aps_moe_weights_register(const aps_moe_weights_desc* desc, void* stream,
                             uint64_t* handle_out);

/* Frees the packed copies.  No reference counterpart: the reference's
 * registry is never freed (src/tensor.cu:1222-1225). */
APS_API int aps_moe_weights_release(uint64_t handle);

/* ---- sizes ------------------------------------------------------------- */

/* Workspace needed by aps_moe_forward / aps_moe_forward_grouped for `rows`
 * tokens with this weight set, and where each array lives in it.  Replaces
 * the reference's grow-only static scratch (src/tensor.cu:1227-1291) and its
 * per-call intermediate Tensors (src/tensor.cu:2835, 2867). */
APS_API int aps_moe_workspace_layout(uint64_t handle, int64_t rows, aps_moe_ws_layout* out);

/* Scratch for aps_moe_dispatch: u32 [ceil(rows/64)][num_experts] (the tile
 * histogram), then one u32 that the call sets to the number of route ids
 * >= num_experts it clamped (the last 4 bytes of this size). */
APS_API size_t aps_moe_dispatch_workspace_size(int64_t rows, int32_t num_experts);

/* ---- stages ------------------------------------------------------------ */

/* Router GEMM logits[rows][E] = x[rows][H] . gate[E][H]^T as one fp32 FMA
 * chain per output, k ascending.  Replaces tensor_ops::matmul_transposed_gpu
 * (reference include/tensor.h:72, src/tensor.cu:3034-3065) on the narrow
 * path it takes for the router (k_matmul_transposed_narrow,
 * src/tensor.cu:2943-3006).  x_dtype: F32 or BF16 (exact upcast). */
APS_API int aps_router_logits(const void* x, int32_t x_dtype, const float* gate,
                      int64_t rows, int32_t hidden, int32_t num_experts,
                      float* logits, void* stream);

/* Quantise + greedy top-2 (reference k_moe_top2, src/tensor.cu:1293-1331;
 * PhiMoE::route, src/layer.cu:69-92).  routes: u8 [rows][2]. */
APS_API int aps_moe_route_top2(const float* logits, int64_t rows, int32_t num_experts,
                       uint8_t* routes, void* stream);

/* Stable counting-sort dispatch (reference k_moe_offsets_work +
 * k_moe_fill_stable, src/tensor.cu:1333-1418).  Outputs counts[E],
 * offsets[E+1], assignment_rows[2*rows], route_positions[2*rows].
 * `scratch` must hold aps_moe_dispatch_workspace_size(rows, E) bytes.
 * Routes are (token, slot) pairs sorted stably by expert, token-major, slot
 * 0 before slot 1.  The reference's routes are always two distinct ids < E;
 * for caller routes that are not, every output index still stays in range:
 * a token whose two slots name one expert takes two consecutive positions
 * of it, and an id >= E is treated as E - 1 and counted into the scratch's
 * last u32 (0 after a call with valid routes). */
APS_API int aps_moe_dispatch(const uint8_t* routes, int64_t rows, int32_t num_experts,
                     uint32_t* counts, uint32_t* offsets,
                     uint32_t* assignment_rows, uint32_t* route_positions,
                     void* scratch, size_t scratch_bytes, void* stream);

/* Grouped expert FFN over the permuted assignments (reference
 * k_moe_pair_silu_8x8 + k_moe_matmul_8x8, src/tensor.cu:1740-1966):
 * y_perm[p] = w2[e] . (silu(w1[e] . x[t]) * (w3[e] . x[t])) for
 * t = assignment_rows[p], p in [offsets[e], offsets[e+1]).
 * act: [2*rows][ffn] scratch of the compute dtype (f32 or bf16; for the
 * fp8 path e4m3 plus act_scale f32 [2*rows]).  y_perm: [2*rows][hidden],
 * f32 for the F32 path, bf16 otherwise.  x_dtype must match the weight
 * set: F32 for the F32 path, BF16 otherwise. */
APS_API int aps_moe_expert_ffn(uint64_t handle, const void* x, int32_t x_dtype, int64_t rows,
                       const uint32_t* offsets, const uint32_t* assignment_rows,
                       void* act, float* act_scale, void* y_perm, void* stream);

/* The two halves of aps_moe_expert_ffn, for callers that schedule or time
 * them separately.  ffn_up replaces k_moe_pair_silu_8x8 (reference
 * src/tensor.cu:1838-1966): act[p] = silu(w1[e] . x[t]) * (w3[e] . x[t]).
 * ffn_down replaces k_moe_matmul_8x8 (src/tensor.cu:1740-1836):
 * y_perm[p] = w2[e] . act[p]. */
APS_API int aps_moe_ffn_up(uint64_t handle, const void* x, int32_t x_dtype, int64_t rows,
                           const uint32_t* offsets, const uint32_t* assignment_rows,
                           void* act, float* act_scale, void* stream);
APS_API int aps_moe_ffn_down(uint64_t handle, const void* act, const float* act_scale,
                             int64_t rows, const uint32_t* offsets, void* y_perm,
                             void* stream);

/* ---- fp8 stages (config C5; no reference counterpart) ------------------ */

/* Per-row e4m3 quantisation: scale[r] = amax(|src[r]|) / 448 (1 for a zero
 * row), dst[r][k] = e4m3(src[r][k] / scale[r]) rounded to nearest even and
 * saturating, for k < n; zero for n <= k < dst_stride.  src bf16 rows with
 * stride src_stride (elements, 16-byte aligned rows); n and dst_stride
 * multiples of 8, dst_stride <= 8192. */
APS_API int aps_quantise_rows_e4m3(const void* src, int64_t src_stride, int32_t n, uint8_t* dst,
                                   int64_t dst_stride, float* scale, int64_t rows, void* stream);

/* The fp8 set's w1||w3 GEMM: act[p] (bf16 [2*rows][ffn]) = silu(g) * u with
 * g = (xq[t] . w1q[e]) * x_scale[t] * w1_scale[e], u likewise (xq: e4m3
 * [rows][hidden] from aps_quantise_rows_e4m3). */
APS_API int aps_moe_ffn_up_fp8(uint64_t handle, const uint8_t* xq, const float* x_scale, int64_t rows,
                               const uint32_t* offsets, const uint32_t* assignment_rows, void* act,
                               void* stream);

/* The fp8 set's w2 GEMM: y_perm[p] (bf16 [2*rows][hidden]) =
 * (actq[p] . w2q[e]) * act_scale[p] * w2_scale[e]; actq: e4m3 [2*rows][ffn
 * rounded up to 128], zero padded (aps_quantise_rows_e4m3 of act). */
APS_API int aps_moe_ffn_down_fp8(uint64_t handle, const uint8_t* actq, const float* act_scale, int64_t rows,
                                 const uint32_t* offsets, void* y_perm, void* stream);

/* Weighted combine (reference k_moe_combine, src/tensor.cu:1968-1988):
 * out[t] = 0.5 * y_perm[route_positions[2t]] + 0.5 * y_perm[route_positions[2t+1]],
 * summed in fp32, rounded once to out_dtype (F32 or BF16). */
APS_API int aps_moe_combine(const void* y_perm, int32_t y_dtype, const uint32_t* route_positions,
                    int64_t rows, int32_t hidden, void* out, int32_t out_dtype,
                    void* stream);

/* ---- whole block ------------------------------------------------------- */

/* Replaces tensor_ops::moe_forward_grouped_gpu (reference
 * include/tensor.h:146-147, src/tensor.cu:2790-2928): routing from
 * precomputed logits [rows][E], then dispatch, expert FFN and combine.
 * x_dtype is the weight set's (F32 / BF16), or F32 with a BF16 weight set
 * (x 16-byte aligned): the FFN then reads a bf16 copy made in the
 * workspace (layout field xq). */
APS_API int aps_moe_forward_grouped(uint64_t handle, const void* x, int32_t x_dtype,
                            const float* router_logits, int64_t rows,
                            void* out, int32_t out_dtype,
                            void* workspace, size_t workspace_bytes, void* stream);

/* Replaces the body of PhiMoE::forward (reference src/layer.cu:113-121):
 * router GEMM (gate [E][H] fp32) + the grouped path above, in one call.
 * The router always reads x in the dtype given (an fp32 x is exact). */
APS_API int aps_moe_forward(uint64_t handle, const void* x, int32_t x_dtype, const float* gate,
                    int64_t rows, void* out, int32_t out_dtype,
                    void* workspace, size_t workspace_bytes, void* stream);

/* aps_moe_forward without a workspace argument: the intermediate arrays
 * live in a static device array of aps_moe_noalloc_scratch_bytes() bytes
 * (96 MiB, one copy per device, held until the process ends), so the call
 * allocates nothing -- for callers that cannot allocate: code under HIP
 * graph capture, serving loops, harnesses that forbid it.  No counterpart
 * in the reference.  Rows whose aps_moe_workspace_layout total exceeds the
 * scratch are refused with APS_ERR_WORKSPACE (up to about 5,500 tokens fit
 * at hidden 4096, ffn 448, bf16: 18.3 KB per token, y and act).  Calls that overlap on one device share the scratch
 * and race: serialise them (one stream, or events). */
APS_API int aps_moe_forward_noalloc(uint64_t handle, const void* x, int32_t x_dtype, const float* gate,
                                    int64_t rows, void* out, int32_t out_dtype, void* stream);
APS_API size_t aps_moe_noalloc_scratch_bytes(void);

/* ---- dense FFN --------------------------------------------------------- */

/* Workspace bytes of aps_mlp_forward for `rows` rows (0 for a bad handle). */
APS_API size_t aps_mlp_workspace_size(uint64_t handle, int64_t rows);

/* Replaces the GPU branch of PhiMLP::forward (reference src/layer.cu:49-67:
 * matmul_pair_silu_gpu, src/tensor.cu:3146-3170 / 967-1057, then
 * matmul_transposed_gpu by w2): out[r] = w2 . (silu(w1 . x[r]) * (w3 . x[r]))
 * for a one-expert weight set.  The fp32 path keeps the reference's
 * accumulation order (k ascending FMA chains, SiLU with exp in double), so
 * it equals the reference bit for bit.  x and out are fp32 for an F32 set,
 * bf16 for a BF16 set. */
APS_API int aps_mlp_forward(uint64_t handle, const void* x, int32_t x_dtype, int64_t rows, void* out,
                            void* workspace, size_t workspace_bytes, void* stream);

/* ---- decoder-layer LayerNorm (the MoE block's input) -------------------- */

/* Replaces tensor_ops::layer_norm_gpu (reference include/tensor.h:86-87,
 * src/tensor.cu:3262-3280, kernel src/tensor.cu:2121-2140): per row of
 * `hidden` fp32 values, mean and variance as single fp32 chains in ascending
 * order (sum += v; var = fma(v - mean, v - mean, var)), inv = 1 / sqrt(var /
 * hidden + eps), y = fma((v - mean) * inv, weight, bias) -- the reference
 * GPU kernel's arithmetic, bit for bit.  hidden % 256 == 0; arrays 16-byte
 * aligned; y must not alias x. */
APS_API int aps_layer_norm(const float* x, const float* weight, const float* bias, int64_t rows,
                           int32_t hidden, float eps, float* y, void* stream);

/* Replaces tensor_ops::add_layer_norm_gpu (reference include/tensor.h:88-90,
 * src/tensor.cu:3282-3295, kernel src/tensor.cu:2144-2178): x += residual
 * in place (one fp32 add per element), then y = LayerNorm(x) as above. */
APS_API int aps_add_layer_norm(float* x, const float* residual, const float* weight, const float* bias,
                               int64_t rows, int32_t hidden, float eps, float* y, void* stream);

/* ---- prompt prefix deduplication (scope row f2) ------------------------- */

/* Replaces tensor_ops::gather_rows_gpu (reference include/tensor.h:115-116 and
 * 138, src/tensor.cu:3379-3386, 3420-3426, kernel k_gather_rows
 * src/tensor.cu:2635-2642): out[i][:] = x[rows[i]][:] for i < count, fp32
 * rows of `hidden` values; rows[] is device memory (the reference's
 * RowIndexBuffer, or its std::vector overload after an upload).  An index
 * >= x_rows gives a row of zeros (the reference does not check; the C++ and
 * Python layers reject such indices before the call).  Any hidden; 16-byte
 * accesses when hidden % 4 == 0 and x, out are 16-byte aligned. */
APS_API int aps_gather_rows(const float* x, int64_t x_rows, int64_t hidden, const uint32_t* rows, int64_t count,
                            float* out, void* stream);

/* The prefix-trie deduplication of PhiTinyMoEModel::generate (reference
 * src/model.cu:44-117), host code, synchronous.  Sequence b is
 * ids[seq_offsets[b] .. seq_offsets[b+1]) (seq_offsets[0] == 0, batch + 1
 * entries).  Writes, for the `*nodes` trie nodes (node ids in creation
 * order, sequence by sequence, as the reference):
 *   token_node[row]  node of packed token row `row` (seq_offsets[batch] entries)
 *   node_token[n]    token id of node n            (capacity seq_offsets[batch])
 *   node_depth[n]    depth = position of node n    (capacity seq_offsets[batch])
 *   node_anc         optional (NULL to skip): [nodes][anc_stride], row n =
 *                    its ancestor chain root .. n, then zeros; anc_stride >=
 *                    the longest sequence.
 * Errors (the reference's std::invalid_argument messages, APS_ERR_ARG):
 * "empty input", "sequence is too long" (length > max_positions), "token out
 * of vocabulary" (outside [0, vocab_size)); batch <= 0 gives APS_ERR_SHAPE
 * "generate received an empty input batch" (a std::runtime_error there). */
APS_API int aps_prefix_dedup(const int32_t* ids, const int64_t* seq_offsets, int64_t batch, int64_t vocab_size,
                             int64_t max_positions, uint32_t* token_node, uint32_t* node_token, uint32_t* node_depth,
                             uint32_t* node_anc, int64_t anc_stride, int64_t* nodes);

/* The ancestor table of aps_prefix_dedup's node_anc, built on the device
 * (the table generate() builds on the host and uploads, reference
 * src/model.cu:64-117): node_anc [nodes][anc_stride], row n = the ancestor
 * chain root .. n, then zeros, equal to the host table bit for bit.  All
 * arrays in device memory: node_parent[n] (the node before n on its
 * sequence; any value for depth-0 nodes), node_depth[n], and run_start[n]
 * = n when node_depth[n] == 0 or node_parent[n] != n - 1, else
 * run_start[n - 1].  anc_stride >= the longest sequence, at most 2^24,
 * and nodes * anc_stride at most 2^38.  Every entry of row n is at most n,
 * whatever the inputs hold.  Asynchronous on `stream`. */
APS_API int aps_prefix_ancestors(const uint32_t* node_parent, const uint32_t* node_depth, const uint32_t* run_start,
                                 int64_t nodes, int64_t anc_stride, uint32_t* node_anc, void* stream);

/* ---- attention over the prefix trie (scope row f4) --------------------- */

/* Replaces Linear::forward's GPU path (reference src/layer.cu:30-42 ->
 * matmul_transposed_bias_gpu / matmul_transposed_gpu, src/tensor.cu:
 * 3034-3143, kernel k_matmul_transposed_8x8 :715-800): y [rows][out] =
 * x [rows][in] . weight [out][in]^T, each output one fp32 FMA chain over k
 * ascending, then + bias[out] when bias is not NULL (the decoder's q/k/v/o
 * projections).  Any in and out (the reference's k_matmul_transposed_tiled
 * fallback, :433-461, serves the shapes its fast kernels do not): in % 16 ==
 * 0, out % 4 == 0 with 16-byte aligned arrays run the vector / matrix-core
 * kernels, other shapes a SIMT kernel with the same chains.  Arrays 4-byte
 * aligned, y not aliasing x. */
APS_API int aps_linear(const float* x, const float* weight, const float* bias, int64_t rows, int32_t in_features,
                       int32_t out_features, float* y, void* stream);
/* Replaces tensor_ops::matmul_pair_bias_gpu (reference include/tensor.h:
 * 77-81, src/tensor.cu:3172-3200), the k and v projections of one input
 * (src/layer.cu:163-166): aps_linear for each of `count` (1..3) outputs of
 * the same x, whose column blocks share one grid (k and v alone would each
 * leave some CUs a third workgroup while others hold two).  Every output
 * is aps_linear's, bit for bit.  Outputs distinct and not x; biases or
 * biases[j] may be NULL. */
APS_API int aps_linear_multi(const float* x, int64_t rows, int32_t in_features, int32_t count,
                             const float* const* weights, const float* const* biases, const int32_t* out_features,
                             float* const* ys, void* stream);

/* The reference's optional tensor-core Linear (built with USE_TC; USE_TC_ALL
 * adds the fourth product and applies it to every attention projection,
 * reference src/layer.cu:16-27).  Not bit-exact: the products are an
 * approximation of the fp32 chain (see aps_linear_tc).
 *
 * Replaces Tensor::prepare_cuda_bf16_weight(with_low_residual = true)
 * (reference include/tensor.h:41-46, src/tensor.cu:124-177): packs weight
 * [out][in] fp32 into bf16 hi = bf16(w) and lo = bf16(w - hi) tile images in
 * `packed` (aps_linear_tc_packed_bytes bytes; 0 for an invalid shape).
 * in % 64 == 0, out % 4 == 0. */
APS_API size_t aps_linear_tc_packed_bytes(int32_t out_features, int32_t in_features);
APS_API int aps_linear_tc_prepare(const float* weight, int32_t out_features, int32_t in_features, void* packed,
                                  size_t packed_bytes, void* stream);
/* The on-the-fly split of x in k_matmul_transposed_bf16_wmma (reference
 * src/tensor.cu:531-543), done once per input: x_split = x_hi [rows][in]
 * then x_lo [rows][in], bf16 (rows * in * 4 bytes). */
APS_API int aps_linear_tc_split(const float* x, int64_t rows, int32_t in_features, void* x_split, void* stream);
/* Replaces matmul_transposed(_bias)_gpu's USE_TC branch (reference
 * src/tensor.cu:3042-3055, kernel k_matmul_transposed_bf16_wmma :514-584,
 * bias after the product :3121-3142): y [rows][out] = x_hi W_hi + x_hi W_lo
 * + x_lo W_hi (+ x_lo W_lo when all_terms), fp32 accumulation on the bf16
 * MFMA, then + bias[out] when bias is not NULL.  The result is within about
 * 1e-5 (all_terms: 1e-6) of the fp32 product relative to its scale, not bit
 * for bit. */
APS_API int aps_linear_tc(const void* x_split, int64_t rows, int32_t in_features, const void* packed,
                          const float* bias, int32_t out_features, int32_t all_terms, float* y, void* stream);
/* PhiAttention's q, k and v projections on the split-bf16 Linear (the
 * reference's q_proj_.forward, then k_proj_ / v_proj_.forward when their
 * weights carry the bf16 copy, src/layer.cu:159-172) in one launch:
 * aps_linear_tc for each of `count` (1..3) outputs of the same x_split,
 * whose column blocks share the grid (the narrow k / v outputs alone would
 * fill few CUs).  Outputs distinct; biases or biases[j] may be NULL. */
APS_API int aps_linear_tc_multi(const void* x_split, int64_t rows, int32_t in_features, int32_t count,
                                const void* const* packed, const float* const* biases, const int32_t* out_features,
                                int32_t all_terms, float* const* ys, void* stream);

/* The RoPE tables of the reference's rope_table (src/tensor.cu:2703-2735),
 * host code: cos/sin [max_seq][head_dim / 2] with inv = powf(theta,
 * (-2 j) / head_dim), cos = cosf(p * inv), sin = sinf(p * inv). */
APS_API int aps_rope_table(int64_t max_seq, int32_t head_dim, float theta, float* cos_out, float* sin_out);

/* Replaces tensor_ops::apply_rope_tree_gpu (reference include/tensor.h:
 * 100-103, src/tensor.cu:3342-3359, kernel k_rope :2180-2197): in place on
 * q [rows][q_heads][head_dim] and k [rows][kv_heads][head_dim], pair (j, j +
 * head_dim / 2) rotated by the table row at row_pos[row]:
 * x0' = fma(x0, c, -(x1 s)), x1' = fma(x1, c, x0 s).  cos_table / sin_table
 * are device copies of aps_rope_table's output; rows whose position is >=
 * max_seq are left unchanged. */
APS_API int aps_rope_tree(float* q, float* k, const uint32_t* row_pos, int64_t rows, int32_t q_heads,
                          int32_t kv_heads, int32_t head_dim, const float* cos_table, const float* sin_table,
                          int64_t max_seq, void* stream);

/* Replaces tensor_ops::attention_tree_gpu (reference include/tensor.h:
 * 109-114, src/tensor.cu:3361-3377, kernel k_attention_tree_gqa4
 * :2407-2633): for each row and query head, softmax attention over the keys
 * anc[row][begin .. pos] (pos = row_pos[row], begin = max(0, pos + 1 -
 * window); the reference's window is SLIDING_WINDOW = 2047), with the
 * reference kernel's arithmetic.  q [rows][q_heads][128], k, v
 * [rows][kv_heads][128], out [rows][q_heads][128], fp32; q_heads = 4 kv_heads
 * ("attention_tree_gpu expects GQA-4"); head_dim 128; k 16-byte aligned.
 * Ancestor entries must be < rows and positions < anc_stride (the kernel
 * clamps them, for memory safety only).  v must be finite: four rows on one
 * ancestor chain are computed together over the union of their windows,
 * and a key outside one row's window enters that row's value products with
 * weight 0, which leaves the result unchanged for a finite value (0 * inf
 * would not); the reference model's activations are finite. */
APS_API int aps_attention_tree(const float* q, const float* k, const float* v, float* out, const uint32_t* row_pos,
                               const uint32_t* anc, int64_t anc_stride, int64_t rows, int32_t q_heads,
                               int32_t kv_heads, int32_t head_dim, int32_t window, void* stream);

/* Replaces tensor_ops::attention_gpu (reference include/tensor.h:
 * 95-98, src/tensor.cu:3318-3340, kernel k_attention_grouped_gqa4
 * :2267-2405): the same attention and arithmetic as aps_attention_tree, over
 * packed token sequences instead of trie nodes (and with its precondition
 * on v: finite values) -- row r of a segment that
 * starts at row seg_offset[r] sits at position seg_pos[r] in it, and its
 * keys are rows seg_offset[r] + begin .. seg_offset[r] + seg_pos[r] (begin =
 * max(0, pos + 1 - window)).  max_seq bounds every segment length (the
 * reference's PackedMeta::max_seq).  q_heads = 4 kv_heads takes the grouped
 * kernel (head_dim 128, k 16-byte aligned); any other layout with q_heads a
 * multiple of kv_heads and head_dim <= 128 the reference's generic kernel's
 * arithmetic (k_attention, :2209-2274: each score one fma chain over d, the
 * same softmax and value chains; any v, no finiteness precondition).  RoPE
 * of packed rows is aps_rope_tree with row_pos = seg_pos. */
APS_API int aps_attention_packed(const float* q, const float* k, const float* v, float* out,
                                 const uint32_t* seg_offset, const uint32_t* seg_pos, int64_t max_seq, int64_t rows,
                                 int32_t q_heads, int32_t kv_heads, int32_t head_dim, int32_t window, void* stream);

/* ---- elementwise fp32 ops of the decoder layer ---------------------------- */

/* a[i] += b[i] for i < n (reference add_inplace_gpu, include/tensor.h:83,
 * src/tensor.cu:3236-3242, kernel k_add :1990-1993). */
APS_API int aps_add_inplace(float* a, const float* b, int64_t n, void* stream);

/* a[i] += bias[i % h] for i < n, n a multiple of h (reference
 * add_bias_inplace_gpu, include/tensor.h:84, src/tensor.cu:3244-3252, kernel
 * k_add_bias :1995-1999). */
APS_API int aps_add_bias_inplace(float* a, const float* bias, int64_t n, int32_t h, void* stream);

/* out[i] = (g / (1 + (float)exp((double)-g))) * up[i], g = gate[i] (reference
 * silu_mul_gpu, include/tensor.h:85, src/tensor.cu:3254-3260, kernel
 * k_silu_mul :2001-2010); out may alias gate or up. */
APS_API int aps_silu_mul(const float* gate, const float* up, float* out, int64_t n, void* stream);

/* x[i] = 0 for i < n by a kernel, so the call may be recorded into a HIP
 * graph (reference zero_gpu, include/tensor.h:82, src/tensor.cu:277-281,
 * a cudaMemsetAsync there). */
APS_API int aps_zero(float* x, int64_t n, void* stream);

/* ---- diagnostics ------------------------------------------------------- */

APS_API const char* aps_moe_last_error(void);
APS_API int aps_moe_abi_version(void);

#ifdef __cplusplus
}
#endif

#endif /* APS_MOE_H */
