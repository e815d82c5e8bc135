/*
 * rqmv: MI355X (gfx950) GGUF quantized matrix-vector library, C ABI.
 *
 * The drop-in boundary for recipe's packed-sum hot path. recipe binds GGUF
 * tensors to projections by name and lowers each to a Contraction (or
 * ExpertIn/ExpertOut/TopK) node whose packed StoredWeight its device code reads
 * (recipe.rs:4532-4832); this library takes over those nodes' storage and
 * arithmetic for batch 1 and small M.
 *
 * Conventions
 *   - Every entry point returns 0 on success and a negative RQMV_E* code on
 *     failure; rqmv_last_error() then names the failure (thread-local). No entry
 *     point aborts the process.
 *   - Weights are owned by the library (device memory, freed by
 *     rqmv_weight_destroy). Activations and outputs are caller-owned device
 *     buffers.
 *   - Work is ordered on the caller's HIP stream (`stream` is a hipStream_t;
 *     NULL = the default stream) and never synchronises the host, except
 *     rqmv_weight_create/unpack, which copy host bytes.
 *   - A weight handle is immutable after creation and may be shared by
 *     threads; launches on one stream are ordered by that stream.
 *   - Activations x are M rows of K values, row m at x + m*ldx elements
 *     (recipe stores positions contiguously per channel, x[k*length + p],
 *     amd-nv-cpu.ll:1161-1165; pass the transpose). Outputs y are fp32, row m
 *     of N values at y + m*ldy. Rows of x start 16-byte aligned (x and
 *     ldx * element size multiples of 16), as device allocations are.
 *   - A NaN or an infinity in an activation row makes that row's outputs
 *     non-finite (NaN where recipe's fp32 sums may give +-inf), never finite;
 *     rqmv_matvec_int8 requires finite activations.
 *   - Accuracy. Weights enter every product at their exact values. Products
 *     of one or two activation rows (and the gguf_moe and decode-step
 *     products) encode each 32-value block of x as 16-bit integers at a step
 *     of (the block's scaling magnitude) / 30583; first, up to four large
 *     values per block (those at or above 1/16 of the largest, taken in
 *     rounds) are set aside and multiplied exactly in fp32. Every other value
 *     is then within 1/60000 of the scaling magnitude, which is at most 16x
 *     the block's fifth largest magnitude: about 2^-12 of it (and 2^-16 of
 *     the block's largest magnitude where nothing is set aside, as for
 *     Gaussian or heavy-tailed activations). Only a block with five or more
 *     outliers on columns whose weights are near zero can lose accuracy
 *     against recipe's fp32 sums. Products of 3 to 32 rows take fp16 x
 *     exactly and fp32 x as an exact-to-2^-22 fp16 pair.
 */
#ifndef RQMV_H
#define RQMV_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* GGML type ids, as recipe's GGUF loader maps them (recipe.rs:9925-9961). */
typedef enum {
    RQMV_F16 = 1,
    RQMV_Q4_0 = 2,
    RQMV_Q8_0 = 8,
    RQMV_Q4_K = 12,
    RQMV_Q6_K = 14
} rqmv_format;

/* Element type of activations. */
typedef enum { RQMV_DTYPE_F32 = 0, RQMV_DTYPE_F16 = 1 } rqmv_dtype;

/* Routing score function (recipe's Scoring: softmax = 0, sigmoid = 1). */
typedef enum { RQMV_SCORE_SOFTMAX = 0, RQMV_SCORE_SIGMOID = 1 } rqmv_scoring;

/* recipe's Activation, by its saved code (Activation::code,
 * recipe.rs:13925-13950), with the programs of activation_program
 * (recipe.rs:22579-22727) and recipe's default constants (Cargo.toml:117-124).
 * RQMV_ACT_GELU_FP16 is Gelu as the llama.cpp profile's gelu table computes
 * it. RQMV_ACT_SCALE multiplies by the factor given beside the code, and
 * RQMV_ACT_PRELU takes that factor as its slope. */
typedef enum {
    RQMV_ACT_LINEAR = 0, RQMV_ACT_COS = 1, RQMV_ACT_EXP = 2, RQMV_ACT_LOG = 3, RQMV_ACT_LN = 4,
    RQMV_ACT_HUBER = 5, RQMV_ACT_TAN = 6, RQMV_ACT_RELU = 7, RQMV_ACT_LEAK = 8, RQMV_ACT_SIGMOID = 9,
    RQMV_ACT_TANH = 10, RQMV_ACT_SELU = 11, RQMV_ACT_GELU = 12, RQMV_ACT_SILU = 13, RQMV_ACT_ELU = 14,
    RQMV_ACT_PRELU = 15, RQMV_ACT_SCALE = 16, RQMV_ACT_SQRT = 17, RQMV_ACT_SOFTPLUS = 18, RQMV_ACT_GELU_FP16 = 32
} rqmv_activation;

enum {
    RQMV_OK = 0,
    RQMV_EINVAL = -1,   /* bad argument, shape or format */
    RQMV_EDEVICE = -2,  /* HIP runtime error */
    RQMV_ENOMEM = -3,   /* device allocation failed */
    RQMV_ESTATE = -4    /* library not initialised for this device */
};

typedef struct rqmv_weight rqmv_weight;

/* Selects and initialises a device; call once per thread that uses it.
 * Replaces the device/queue set-up of recipe's HSA runtime
 * (recipe.rs:28007-28612, Gpu::open). */
int rqmv_init(int device);

/* The last failure on the calling thread, or "" (recipe.rs:13416-13433). */
const char* rqmv_last_error(void);

/* Uploads rows x cols weights given as GGUF block bytes (row-major: row r is
 * cols/block consecutive blocks, recipe.rs:9875-9889), repacked into the
 * kernels' layout. Replaces StoredWeight + Buffer::fill_weights with
 * row_interleave (recipe.rs:15859-16069, 26980-27010, 3162-3212).
 * cols is a whole number of blocks (32 for Q8_0/Q4_0, 256 for Q4_K/Q6_K) and
 * a multiple of 32; F16 rows are packed in 64-value chunks, so an F16 weight
 * (a router) needs a multiple of 64. Other widths are RQMV_EINVAL. */
int rqmv_weight_create(int format, int64_t rows, int64_t cols, const void* gguf_bytes, size_t nbytes,
                       rqmv_weight** out);

/* An expert bank: `experts` consecutive rows x cols matrices, as GGUF stores
 * ffn_{gate,up,down}_exps shaped [cols, rows, experts] (recipe.rs:9861-9868,
 * 18286-18292). */
int rqmv_expert_bank_create(int format, int64_t experts, int64_t rows, int64_t cols, const void* gguf_bytes,
                            size_t nbytes, rqmv_weight** out);

int rqmv_weight_destroy(rqmv_weight* weight);

/* Shape, format and device footprint of a weight (experts = 1 for a plain one). */
int rqmv_weight_info(const rqmv_weight* weight, int* format, int64_t* rows, int64_t* cols, int64_t* experts,
                     size_t* device_bytes);

/* Copies the weight back to host memory as GGUF block bytes (the inverse of
 * the repack; nbytes must equal the GGUF size). Synchronises the device. */
int rqmv_weight_unpack(const rqmv_weight* weight, void* gguf_bytes, size_t nbytes);

/* Writes every weight as fp32, rows x cols (x experts) in GGUF order, each
 * equal to recipe's reference dequantization rounded to fp32
 * (HostQuantOps, recipe.rs:3687-3833, 3973-4057). */
int rqmv_weight_dequantize(const rqmv_weight* weight, float* out_dev, void* stream);

/* y = W x for M activation rows (Gguf::contract, recipe.rs:17130; a packed
 * Contraction node, recipe.rs:4532-4604 / amd-nv-cpu.ll:2674-3126). */
int rqmv_matvec(const rqmv_weight* weight, const void* x_dev, int x_dtype, int m, int64_t ldx, float* y_dev,
                int64_t ldy, void* stream);

/* rqmv_matvec with two HIP events (hipEvent_t, either may be NULL) that the
 * kernel dispatch itself records at its start and at its completion, for
 * measuring kernel time without host launch overhead. No counterpart in the
 * reference; for benchmarks and profilers. */
int rqmv_matvec_timed(const rqmv_weight* weight, const void* x_dev, int x_dtype, int m, int64_t ldx, float* y_dev,
                      int64_t ldy, void* stream, void* start_event, void* stop_event);

/* y = W_e x with expert `expert` of a bank (Gguf::expert, recipe.rs:17135). */
int rqmv_expert_matvec(const rqmv_weight* bank, int64_t expert, const void* x_dev, int x_dtype, int m, int64_t ldx,
                       float* y_dev, int64_t ldy, void* stream);

/* The gguf_moe block (recipe.rs:14722, lowered at 23415-23459): router,
 * top-k routing, routed gated experts and an optional shared expert. Every
 * argument of gguf_moe(experts, top_k, hidden, activation, scoring,
 * renormalize, shared, scale, selection_bias) has a field here: experts and
 * hidden are the banks' shapes; shared is SharedExpert::None (no shared
 * weights), ::Ungated (shared weights, shared_gate_inp NULL: weight one) or
 * ::Gated { gate } (shared_gate_inp and shared_gate_activation = gate). */
typedef struct {
    const rqmv_weight* router;      /* F16, experts x d_model (ffn_gate_inp) */
    const rqmv_weight* gate_exps;   /* bank: experts x hidden x d_model (ffn_gate_exps) */
    const rqmv_weight* up_exps;     /* bank: experts x hidden x d_model (ffn_up_exps) */
    const rqmv_weight* down_exps;   /* bank: experts x d_model x hidden (ffn_down_exps) */
    const rqmv_weight* shared_gate_inp; /* F16, 1 x d_model (ffn_gate_inp_shexp) or NULL */
    const rqmv_weight* gate_shexp;  /* hidden_shared x d_model, or NULL for no shared expert */
    const rqmv_weight* up_shexp;
    const rqmv_weight* down_shexp;  /* d_model x hidden_shared */
    int top_k;
    int scoring;        /* rqmv_scoring */
    int renormalize;    /* divide the kept weights by their total */
    float scale;        /* routed weight scale (1 = none) */
    int activation;     /* rqmv_activation of every expert: act(gate x) * (up x) (lower_gated,
                           recipe.rs:23279-23286); RQMV_ACT_SILU for llama-style experts.
                           Code 0 is RQMV_ACT_LINEAR: a zero-initialised struct gets linear
                           experts and a linear shared gate, so set both codes explicitly
                           (RQMV_ACT_SILU and RQMV_ACT_SIGMOID for llama-style blocks) */
    int shared_gate_activation; /* rqmv_activation of the shared gate (SharedExpert::Gated's gate) */
    float activation_factor;    /* RQMV_ACT_SCALE's constant, RQMV_ACT_PRELU's slope (else unused);
                                   must be finite when either code uses it, else RQMV_EINVAL */
    const float* selection_bias; /* device, experts fp32 values (exp_probs_b.bias) or NULL: the top-k
                                    key becomes the expert's probability plus its bias, the weights
                                    stay those of the unbiased scores (topk_key, amd-nv-cpu.ll:4653-4660) */
} rqmv_moe_params;

/* Device workspace bytes rqmv_moe needs for one position. It also checks the
 * parameters: the banks are quantized, the hidden width and d_model are
 * multiples of the bank format's 16-byte-part chunk (32 values for Q8_0, 64
 * for Q4_0, a superblock's 256 for Q4_K/Q6_K), the router is F16 (d_model a
 * multiple of 64), and top is in 1..min(64, experts) with at most 2048 experts;
 * otherwise RQMV_EINVAL. */
int rqmv_moe_workspace_size(const rqmv_moe_params* params, size_t* bytes);

/* One position: x (d_model, f16 or f32) -> y (d_model, fp32). The routing
 * weights (experts floats, zero off the top-k) are written to route_dev when
 * it is not NULL. `workspace` is a device buffer of rqmv_moe_workspace_size
 * bytes that the call may overwrite. */
int rqmv_moe(const rqmv_moe_params* params, const void* x_dev, int x_dtype, float* y_dev, float* route_dev,
             void* workspace, size_t workspace_bytes, void* stream);

/* m positions at once (a prefill batch; recipe runs gguf_moe over every
 * position of a step, each routed on its own): position p reads x_dev + p*ldx
 * elements and writes y_dev + p*ldy; its routing weights go to route_dev +
 * p*experts when route_dev is not NULL. The workspace holds m times
 * rqmv_moe_workspace_size bytes. Still three launches for the whole batch. */
int rqmv_moe_batch(const rqmv_moe_params* params, const void* x_dev, int x_dtype, int m, int64_t ldx, float* y_dev,
                   int64_t ldy, float* route_dev, void* workspace, size_t workspace_bytes, void* stream);

/* rqmv_moe_batch without a workspace argument, for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc). No counterpart in the reference. The
 * workspace is the library's own 1 MiB scratch array, one per GPU, held until
 * the process ends: m positions fit when m * rqmv_moe_workspace_size bytes
 * <= 1 MiB (the 2048 x 512, 256-expert top-8 block takes about 20 KiB per
 * position), else RQMV_EINVAL. The call allocates nothing. Every call on one
 * GPU shares that GPU's scratch: calls that overlap on it (other streams,
 * other threads) race, so order them. */
int rqmv_moe_batch_noalloc(const rqmv_moe_params* params, const void* x_dev, int x_dtype, int m, int64_t ldx,
                           float* y_dev, int64_t ldy, float* route_dev, void* stream);

/* Decode-step helpers. They have no counterpart at the matrix-vector
 * boundary: they run the rest of a decoder layer on the device between the
 * projections, for the end-to-end single-token decode, with the semantics of
 * recipe's attention block and feed-forward (lower_attention,
 * recipe.rs:23056-23150; silu(gate) * up, 23279-23286, 22662-22668). All
 * pointers are device pointers; `pos` points to a device int32 holding the
 * token's position (so that a captured step replays at the next position
 * after rqmv_advance). Activations are fp32; the KV cache is fp16, laid out
 * [kv head][position][head_dim] with max_ctx positions per head. */

/* x += delta (delta may be NULL); out = x / sqrt(mean(x^2) + eps) * weight. */
int rqmv_add_rmsnorm(float* x, const float* delta, const float* weight, int n, float eps, float* out, void* stream);

/* NeoX rotary on the q and k heads of qkv ([q | k | v] heads of head_dim, in
 * place; pair i turns by pos * base^(-2i/head_dim)), then the rotated keys and
 * the values are stored in the caches at pos (nothing is stored when pos is
 * outside 0..max_ctx-1). */
int rqmv_rope_kv(float* qkv, const int* pos, int q_heads, int kv_heads, int head_dim, double base, void* k_cache,
                 void* v_cache, int max_ctx, void* stream);

/* Grouped-query attention of one query (q_heads x head_dim) over positions
 * 0..min(pos, max_ctx - 1) of the cache: softmax(q k / sqrt(head_dim)) v per
 * query head. head_dim is 64, 128 or 256; at most 8 query heads share a kv
 * head; max_ctx is at most 65536; q, the caches, the workspace and out are
 * 16-byte aligned. Two launches (per-chunk partial results in the workspace,
 * then their merge); calls sharing a workspace must not overlap. */
int rqmv_attention_workspace_size(int q_heads, int kv_heads, int head_dim, int max_ctx, size_t* bytes);
int rqmv_attention(const float* q, const void* k_cache, const void* v_cache, const int* pos, int q_heads, int kv_heads,
                   int head_dim, int max_ctx, void* workspace, size_t workspace_bytes, float* out, void* stream);

/* table[p][i] = (cos, sin) of p * base^(-2i/head_dim) for p < rows, i <
 * head_dim / 2, as fp32 pairs (rows x head_dim floats), the angle and its
 * cosine and sine taken in f64 as rqmv_rope_kv takes them. */
int rqmv_rope_table(float* table, int head_dim, double base, int rows, void* stream);

/* rqmv_rope_kv and rqmv_attention in one: qkv holds the unrotated [q | k | v]
 * heads; the queries and the new key are rotated with `rope_table` (max_ctx
 * rows from rqmv_rope_table), the new key and value are stored in the caches
 * at pos and attended to along with positions 0..pos-1. qkv is not modified.
 * Positions at or past max_ctx are outside the cache: nothing is stored and
 * the rotation uses the table's last row. */
int rqmv_attention_rope(const float* qkv, const float* rope_table, void* k_cache, void* v_cache, const int* pos,
                        int q_heads, int kv_heads, int head_dim, int max_ctx, void* workspace, size_t workspace_bytes,
                        float* out, void* stream);

/* out[i] = silu(gate_up[i]) * gate_up[n + i]. */
int rqmv_silu_mul(const float* gate_up, int n, float* out, void* stream);

/* *out = the index of the largest value (the lowest index on a tie; NaNs
 * are skipped). Two launches (per-slice bests in the workspace, then their
 * reduction); calls sharing a workspace must not overlap. */
int rqmv_argmax_workspace_size(size_t* bytes);
int rqmv_argmax(const float* values, int n, int* out, void* workspace, size_t workspace_bytes, void* stream);

/* out = table[token mod rows] (rows x n fp32): the next token's embedding. */
int rqmv_embed_row(const float* table, int rows, int n, const int* token, float* out, void* stream);

/* A gate and an up projection of one width stored as one weight of 2 x rows
 * rows, (gate_i, up_i) interleaved, for the fused SiLU-GLU epilogue. Each of
 * gate_gguf and up_gguf is rows x cols GGUF blocks (ffn_gate, ffn_up). Plain
 * rqmv_matvec on it writes the 2 x rows products in that interleaved order. */
int rqmv_glu_weight_create(int format, int64_t rows, int64_t cols, const void* gate_gguf, const void* up_gguf,
                           size_t nbytes_each, rqmv_weight** out);

/* A decode-step product with its neighbours folded in (one fp32 activation
 * row, a plain quantized weight):
 *   prologue (norm_weight != NULL): the product reads u = x + delta (delta
 *     may be NULL), normalised: u_i * norm_weight_i / sqrt(sum u^2 / cols +
 *     eps); when x_out is not NULL, u itself is written there (the updated
 *     residual stream; x_out must differ from x and delta);
 *   epilogue RQMV_EPI_PLAIN: y = W u';
 *   epilogue RQMV_EPI_GLU (a rqmv_glu_weight_create weight): y_i =
 *     silu(gate_i u') * (up_i u'), silu(v) = v * 0.5 (tanh(v / 2) + 1).
 * recipe runs these as separate nodes (the residual add, Normalize,
 * Contraction and the SiLU-GLU product: recipe.rs:23190-23210, 4532-4604,
 * 23279-23286); the fusion saves their launches and activation round trips. */
enum { RQMV_EPI_PLAIN = 0, RQMV_EPI_GLU = 1 };
typedef struct {
    const float* norm_weight;
    float eps;
    const float* delta;
    float* x_out;
    int epilogue;
} rqmv_fusion;
int rqmv_matvec_fused(const rqmv_weight* weight, const float* x_dev, float* y_dev, const rqmv_fusion* fusion,
                      void* stream);

/* recipe's int(8) sum: the product recipe computes when a precision profile
 * declares `sum = "int8"` (the default profile, step 32, and the llama.cpp
 * profile, step 256; Cargo.toml:143-201) on a backend with int8 dots
 * (contraction_forward_gemv_wave_body, amd-nv-cpu.ll:1231-2241). Each of the
 * m fp32 activation rows (row i at x + i*ldx) is rounded to Q8 records (one
 * fp32 step per `step` inputs, a signed byte per input); the block dots run
 * on v_dot4_i32_i8 and the fp32 tail in recipe's order, so y[i*ldy + n] has
 * the bits recipe's 32-lane GPU backends produce. Formats Q4_K, Q6_K, Q8_0,
 * Q4_0 (an expert bank counts as experts x rows rows). At step 256 a Q4_K
 * position before the last m % 4 folds each block in four quarters, as
 * llama.cpp's batched kernel does; flags RQMV_INT8_TAIL folds the last
 * position whole (recipe's model tail, amd-nv-cpu.ll:1716-1722). x must be
 * finite, 16-byte aligned, ldx a multiple of 4; about cols * 1.14 bytes of
 * LDS hold the records. */
enum { RQMV_INT8_TAIL = 1 };
int rqmv_matvec_int8(const rqmv_weight* weight, const float* x_dev, int m, int64_t ldx, float* y_dev, int64_t ldy,
                     int step, int flags, void* stream);

/* The gfx950 row of recipe's capability table (FormatCapability rows and
 * resolve_capability, recipe.rs:2646-2745): for a compute format named as
 * recipe names it ("int4", "int8", "int16", "int32", "fp8", "fp16", "fp32",
 * "fp64", "bf16", "tf32"), the vector and matrix instructions this library
 * uses (static strings; NULL where there is none). A format with neither is
 * an error whose message lists the formats that have each, as recipe's. */
int rqmv_capability(const char* format, const char** vector, const char** matrix);

/* A weight in the storage recipe's int(8) profile gives it (finish_int_sums
 * and requantize_bound, recipe.rs:22327-22437): Q4_K and Q8_0 are kept as they
 * are; F16, Q4_0 and Q6_K are re-encoded to Q8_0 as recipe's load kernel does
 * (the device Q8_0 quantizer, recipe.rs:8016-8080: per 32 values scale =
 * |first largest| / 127, code = trunc(v / scale +- 0.5) clamped, d = fp16
 * of the scale), here on the host, once. rqmv_weight_info reports the stored
 * format. experts = 1 for a plain weight. */
int rqmv_weight_create_int8(int format, int64_t experts, int64_t rows, int64_t cols, const void* gguf_bytes,
                            size_t nbytes, rqmv_weight** out);

/* That re-encoding alone, host to host: rows x cols GGUF weights of `format`
 * (F16, Q8_0, Q4_0 or Q6_K) -> rows * cols / 32 Q8_0 blocks (34 bytes each). */
int rqmv_requantize_q8_0_host(int format, int64_t rows, int64_t cols, const void* gguf_bytes, size_t nbytes,
                              void* out);

/* The Q8 records of one activation row of k inputs (k a multiple of 32, x
 * 16-byte aligned) that rqmv_matvec_int8 forms in LDS (amd-nv-cpu.ll:1408-1500): d_dev[k/32] steps
 * (one value per `step` inputs, repeated per 32) and codes_dev[k] bytes. */
int rqmv_q8_records(const float* x_dev, int64_t k, int step, float* d_dev, int8_t* codes_dev, void* stream);

/* *pos += 1 on the device (the last launch of a captured decode step). */
int rqmv_advance(int* pos, void* stream);

/* GGUF v3 files (recipe's mod gguf, recipe.rs:9783-10327; Gguf::open 10069,
 * tensor / value / data 10141-10174). The file is mapped read-only; a split
 * model (<prefix>-<n>-of-<count>.gguf with split.count) is opened whole from
 * its first shard. Names and strings returned stay valid until
 * rqmv_gguf_close. Shapes are in GGML order: dims[0] is the row width. None
 * of these touch a device except rqmv_gguf_weight_create. */
typedef struct rqmv_gguf rqmv_gguf;
int rqmv_gguf_open(const char* path, rqmv_gguf** out);
int rqmv_gguf_close(rqmv_gguf* file);
int rqmv_gguf_tensor_count(const rqmv_gguf* file, int64_t* count);
/* dims holds up to 8 entries. */
int rqmv_gguf_tensor_info(const rqmv_gguf* file, int64_t index, const char** name, int* ggml_type, int* n_dims,
                          int64_t* dims, size_t* nbytes);
int rqmv_gguf_find_tensor(const rqmv_gguf* file, const char* name, int64_t* index);
/* The tensor's bytes in the mapped file, in its GGML block layout. */
int rqmv_gguf_tensor_data(const rqmv_gguf* file, int64_t index, const void** data, size_t* nbytes);
int rqmv_gguf_metadata_count(const rqmv_gguf* file, int64_t* count);
/* Key `index` (file order) and its GGUF value type (0..12). */
int rqmv_gguf_metadata_key(const rqmv_gguf* file, int64_t index, const char** key, int* value_type);
/* A nonnegative integer of any width (GgufValue::integer), a float (F32 or
 * F64), a string; arrays by element. */
int rqmv_gguf_get_int(const rqmv_gguf* file, const char* key, int64_t* out);
int rqmv_gguf_get_float(const rqmv_gguf* file, const char* key, double* out);
int rqmv_gguf_get_string(const rqmv_gguf* file, const char* key, const char** out);
int rqmv_gguf_get_array(const rqmv_gguf* file, const char* key, int* element_type, int64_t* count);
int rqmv_gguf_get_array_int(const rqmv_gguf* file, const char* key, int64_t index, int64_t* out);
int rqmv_gguf_get_array_string(const rqmv_gguf* file, const char* key, int64_t index, const char** out);
/* A device weight from a named tensor, straight from the mapped bytes: [k, n]
 * is n rows of k, [k, n, experts] an expert bank (recipe.rs:18286-18292). */
int rqmv_gguf_weight_create(const rqmv_gguf* file, const char* name, rqmv_weight** out);

/* Host-only loader functions (no device needed): the repacked layout's size
 * and the repack / unpack themselves, for inspection and testing. */
int rqmv_layout_bytes(int format, int64_t rows, int64_t cols, size_t* bytes);
int rqmv_repack_host(int format, int64_t rows, int64_t cols, const void* gguf_bytes, void* out);
int rqmv_unpack_host(int format, int64_t rows, int64_t cols, const void* in, void* gguf_bytes);

#ifdef __cplusplus
}
#endif
#endif
