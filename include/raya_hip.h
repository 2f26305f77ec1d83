/*
 * raya_hip.h: C ABI of libraya_hip.so, the MI355X (gfx950) backend for raya's
 * block-local attention hot path and the encoder GEMMs.
 *
 * Plain pointers and sizes only.  Every entry point returns RAYA_OK (0) or one
 * of the RAYA_ERR_* codes; details of the last failure on the calling thread
 * are in raya_last_error().  Entry points never abort the process on bad
 * arguments.
 *
 * Citations are to joaoajmatos/raya (Rust).
 */
#ifndef RAYA_HIP_H
#define RAYA_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Error codes.  SHAPE, LENGTH and UNSUPPORTED are the three variants of
 * KernelError (crates/raya-kernels/src/attention.rs:8-20); DEVICE carries a HIP
 * runtime failure, which the reference (CPU only) never produces. */
#define RAYA_OK 0
#define RAYA_ERR_SHAPE 1
#define RAYA_ERR_LENGTH 2
#define RAYA_ERR_UNSUPPORTED 3
#define RAYA_ERR_DEVICE 4

/* Mask kinds: Mask::{Block3, Window64, Full, Sliding(w)}
 * (crates/raya-kernels/src/attention.rs:22-35) plus BlockDiag(b), where a query
 * in block i/b sees only the keys of its own block (no reference counterpart). */
#define RAYA_MASK_BLOCK3 0
#define RAYA_MASK_WINDOW64 1
#define RAYA_MASK_FULL 2
#define RAYA_MASK_SLIDING 3
#define RAYA_MASK_BLOCKDIAG 4

/* The reference's fixed block (attention.rs:4) and window (attention.rs:6). */
#define RAYA_BLOCK 128
#define RAYA_WINDOW 64

/* AttnShape, attention.rs:72-84: buffers are [heads][seq][head_dim] f32. */
typedef struct raya_attn_shape {
    uint64_t heads;
    uint64_t seq;
    uint64_t head_dim;
} raya_attn_shape;

/* AttnParams, attention.rs:86-93, with the Mask enum flattened into
 * (mask_kind, mask_arg): mask_arg is w for Sliding(w), b for BlockDiag(b) and
 * ignored otherwise.  block must be RAYA_BLOCK, as the reference's validate
 * requires (attention.rs:153-158). */
typedef struct raya_attn_params {
    int32_t mask_kind;
    float scale;
    uint64_t mask_arg;
    uint64_t block;
    uint64_t valid_len;
} raya_attn_params;

/* Details of the last failure on the calling thread.  For RAYA_ERR_LENGTH,
 * buffer/got/expected are the fields of KernelError::Length; message is the
 * error's Display text as the reference formats it. */
typedef struct raya_error {
    int32_t code;
    char buffer[8];
    uint64_t got;
    uint64_t expected;
    char message[512];
} raya_error;

const raya_error *raya_last_error(void);

/* Stable names for bench output, like AttentionKernel::name (attention.rs:114)
 * and GemmBackend::name (gemm.rs:3). */
const char *raya_attention_name(void);
const char *raya_gemm_name(void);

/* How this library was built, fixed at build time as the reference's
 * BenchMetadata fields rustc and git_commit are (crates/raya-kernels/src/
 * meta.rs:12-27, build.rs): lines "arch=...", "compiler=...", "commit=..."
 * and "flags=...", "unknown" where the build could not tell. */
const char *raya_build_info(void);

/* AttentionKernel::attend (crates/raya-kernels/src/attention.rs:113-125) on
 * host slices: validates like validate() (attention.rs:128-170) plus the
 * HIP kernel's limits (head_dim <= 256), copies q/k/v to the current device,
 * runs the fused kernel, copies out back and synchronises.  out is fully
 * overwritten; rows >= valid_len are exact zeros. */
int raya_attend(const raya_attn_shape *shape, const raya_attn_params *params,
                const float *q, size_t q_len, const float *k, size_t k_len,
                const float *v, size_t v_len, float *out, size_t out_len);

/* Per-stage totals of the attention kernel in shader clock cycles, summed over
 * waves: the device counterpart of StageTimes (crates/raya-kernels/src/tiled/
 * stages.rs:3-31).  As there, only the shares are meaningful: waves of one
 * compute unit overlap, so the sums exceed the kernel's duration. */
typedef struct raya_stage_cycles {
    uint64_t qk;        /* S^T = K Q^T of each tile (the reference's qk_ns) */
    uint64_t softmax;   /* masking, running max and sum, rescale, exp (softmax_ns) */
    uint64_t pv;        /* O^T += V^T P^T (pv_ns) */
    uint64_t load_wait; /* K/V load issue, waits for them and the workgroup barriers
                           (no reference counterpart: its loads are inside the stages) */
    uint64_t tiles;     /* computed tiles of 16 query rows x 64 keys (tiles) */
} raya_stage_cycles;

/* Tiled::attend_with_stages (crates/raya-kernels/src/tiled/mod.rs:61-126) on
 * host slices: raya_attend through an instrumented copy of the kernel that
 * reads the shader clock around each tile's stages (raya_attend itself carries
 * no timing code).  *stages receives this call's totals; out equals
 * raya_attend's bit for bit. */
int raya_attend_with_stages(const raya_attn_shape *shape, const raya_attn_params *params,
                            const float *q, size_t q_len, const float *k, size_t k_len,
                            const float *v, size_t v_len, float *out, size_t out_len,
                            raya_stage_cycles *stages);

/* raya_attend without device allocation.  No counterpart in the reference: for
 * callers that cannot allocate device memory (serving loops, harnesses that
 * forbid hipMalloc).  The operands are staged in a static device array of four
 * slots of RAYA_STATIC_ATTEND_MAX_NUMEL floats (64 MiB on every device the
 * library runs on, held until the process ends) instead of raya_attend's
 * grow-only workspace, and the copies and the launch run on `stream` (a
 * hipStream_t of the current device; NULL is the null stream), which is
 * synchronised before the call returns.  Same checks and errors as raya_attend,
 * then RAYA_ERR_UNSUPPORTED when heads * seq * head_dim exceeds
 * RAYA_STATIC_ATTEND_MAX_NUMEL or the stream belongs to another device.  Each
 * device's array is shared by every call on that device; those calls are
 * serialised on a per-device lock, so they never overlap.  Nothing in it needs
 * clearing: each call overwrites the q, k, v and out slots it uses. */
#define RAYA_STATIC_ATTEND_MAX_NUMEL 4194304
int raya_attend_static(const raya_attn_shape *shape, const raya_attn_params *params, const float *q,
                       size_t q_len, const float *k, size_t k_len, const float *v, size_t v_len, float *out,
                       size_t out_len, void *stream);

/* Row strides of one operand in floats.  All zero selects the dense
 * [batch][heads][seq][head_dim] layout. */
typedef struct raya_attn_layout {
    int64_t batch_stride;
    int64_t head_stride;
    int64_t row_stride;
} raya_attn_layout;

/* A batch of sequences on the device: batch trait calls in one launch, each
 * sequence with its own valid length.  No reference counterpart (the trait
 * takes one sequence). */
typedef struct raya_attn_batch {
    uint64_t batch;
    uint64_t heads;
    uint64_t seq;
    uint64_t head_dim;
    int32_t mask_kind;
    float scale;
    uint64_t mask_arg;
    uint64_t block;
    raya_attn_layout q, k, v, out;
} raya_attn_batch;

/* Device pointers, asynchronous on `stream` (a hipStream_t; NULL is the null
 * stream).  valid_len is a device array of batch int32 values; values outside
 * [0, seq] are clamped into it.  Pointers must be 16-byte aligned and strides
 * multiples of 4 floats. */
int raya_attend_batched(const raya_attn_batch *desc, const int32_t *valid_len,
                        const float *q, const float *k, const float *v, float *out,
                        void *stream);

/* raya_attend_with_stages for a device batch: raya_attend_batched through the
 * instrumented kernel.  `stages` is a device pointer; the totals are ADDED
 * to it (StageTimes::merge), so zero it before the first call.  Outputs equal
 * raya_attend_batched's bit for bit.  Asynchronous on `stream`. */
int raya_attend_batched_stages(const raya_attn_batch *desc, const int32_t *valid_len,
                               const float *q, const float *k, const float *v, float *out,
                               raya_stage_cycles *stages, void *stream);

/* GemmBackend::matmul_nt (crates/raya-kernels/src/gemm.rs:2-11) on host
 * slices: out[m][n] = sum_t a[m][t] * b[n][t].  Length mismatches return
 * RAYA_ERR_LENGTH with buffer "a", "b" or "out" and the reference's panic text
 * ("a must be [m, k]", gemm.rs:23-25) as message; the caller re-raises them. */
int raya_matmul_nt(float *out, size_t out_len, const float *a, size_t a_len,
                   const float *b, size_t b_len, uint64_t m, uint64_t n, uint64_t k);

/* GEMM epilogues: y = acc + bias; y = activation(y); out = y + residual.
 * GELU is the exact erf form of ops::gelu (crates/raya-core/src/ops.rs:35-38),
 * ReLU is ops::relu (ops.rs:41-43).  GEGLU follows the gated MLP of
 * encoder::layer (crates/raya-core/src/encoder.rs:139-146): b has 2n rows and
 * out[i][j] = gelu(y[i][j]) * y[i][n + j]. */
#define RAYA_EPI_NONE 0
#define RAYA_EPI_GELU 1
#define RAYA_EPI_RELU 2
#define RAYA_EPI_GEGLU 3

typedef struct raya_gemm_epilogue {
    int32_t activation;    /* RAYA_EPI_* */
    int32_t reserved;      /* must be 0 */
    const float *bias;     /* device [n] ([2n] for GEGLU) or NULL */
    const float *residual; /* device [m][ldr] or NULL; may alias out when ldr == ldo */
    int64_t ldr;
    /* Residual + LayerNorm across two GEMMs, the pre-LN encoder's
     * h += x Wo^T; LayerNorm(h) Wi^T (crates/raya-core/src/encoder.rs:127-146, whose
     * ops::layer_norm, ops.rs:51-74, is a pass of its own there):
     *  - out_row_stats: device [m][n / 64][4] floats or NULL.  Per row and 64-column chunk
     *    of out (after the residual add), the statistics raya_row_norm_stats turns into
     *    the row's LayerNorm mean and 1 / sqrt(var + eps).  n a multiple of 64; not GEGLU.
     *  - in_row_stats: device [m][4] floats (raya_row_norm_stats' output) or NULL.  The
     *    rows of a are normalised before the product: out = epilogue(LayerNorm(a) b^T),
     *    with b the weight whose columns the caller has multiplied by the norm's gain
     *    (b[j][t] = gain[t] W[j][t]) and in_weight_sums its row sums (raya_weight_row_sums,
     *    device [n], [2n] for GEGLU); a norm bias beta enters as the GEMM bias W beta.  A
     *    row whose mean lies more than one standard deviation from zero is centred before
     *    the contraction, as ops::layer_norm subtracts the mean before scaling; for the
     *    others the mean comes out afterwards through the row sums.
     * Both need the ring kernel: k a multiple of 16, lda, ldb, ldo (and ldr) multiples of
     * 4 floats, 16-byte aligned a, b and out (and residual); otherwise RAYA_ERR_UNSUPPORTED. */
    float *out_row_stats;
    const float *in_row_stats;
    const float *in_weight_sums;
} raya_gemm_epilogue;

/* Device-pointer GEMM with a fused epilogue (ep may be NULL: plain product),
 * asynchronous on `stream`.  Leading dimensions are in floats.  No reference
 * counterpart: linear() (ops.rs:91-109) applies bias and activations on the
 * host after matmul_nt. */
int raya_matmul_nt_device(float *out, int64_t ldo, const float *a, int64_t lda, const float *b,
                          int64_t ldb, uint64_t m, uint64_t n, uint64_t k,
                          const raya_gemm_epilogue *ep, void *stream);

/* Each row's LayerNorm statistics (mean and 1 / sqrt(var + eps), var the biased variance,
 * in f64 as ops::layer_norm computes them, crates/raya-core/src/ops.rs:51-74) from the
 * chunk statistics a GEMM wrote to out_row_stats for an output of width n (a multiple of
 * 64): chunk_stats [rows][n / 64][4] -> row_stats [rows][4], both device, for a later
 * GEMM's in_row_stats.  eps finite and >= 0.  Asynchronous on `stream`. */
int raya_row_norm_stats(const float *chunk_stats, uint64_t rows, uint64_t n, float eps, float *row_stats,
                        void *stream);

/* sums[j] = sum_t b[j][t] over t < k, in f64 rounded once to f32, for j < rows: the weight
 * row sums a GEMM with in_row_stats needs (computed once per folded weight).  Device
 * pointers, ldb >= k floats; asynchronous on `stream`. */
int raya_weight_row_sums(const float *b, int64_t ldb, uint64_t rows, uint64_t k, float *sums, void *stream);

/* ---- A post-LN encoder layer ----------------------------------------------------------------
 *
 * No counterpart in the reference, whose encoder layer is pre-LN (encoder::layer,
 * crates/raya-core/src/encoder.rs:96-152): BERT's layer, i.e. nn.TransformerEncoderLayer with
 * norm_first=False, GELU (erf) and biases, as a block-local encoder layer is usually written:
 *   y1  = LayerNorm1(x + Attn(x Wqkv^T + bqkv) Wo^T + bo)
 *   out = LayerNorm2(y1 + gelu(y1 W1^T + b1) W2^T + b2)
 * Attention uses the mask (mask_kind, mask_arg) and the per-sequence valid lengths, scale
 * 1/sqrt(head_dim); its rows at or beyond valid_len are zero, as Naive::attend's.  Weights are
 * device pointers in nn.Linear's [out_features][in_features] layout (wqkv: q, k and v stacked,
 * [3 hidden][hidden]); any bias may be NULL (zero).  LayerNorm eps is ln_eps (finite, >= 0). */
typedef struct raya_postln_layer {
    uint64_t batch, seq, hidden, heads, ffn;
    int32_t mask_kind;
    int32_t reserved; /* must be 0 */
    uint64_t mask_arg;
    float ln_eps;
    const float *wqkv, *bqkv, *wo, *bo, *ln1_w, *ln1_b, *w1, *b1, *w2, *b2, *ln2_w, *ln2_b;
} raya_postln_layer;

/* Device workspace the layer needs (qkv, context, sums, y1, feed-forward activations: batch *
 * seq * (6 hidden + ffn) floats), or 0 when the layer description is invalid. */
uint64_t raya_postln_workspace_bytes(const raya_postln_layer *layer);

/* x and out: device [batch][seq][hidden] fp32 (16-byte aligned), valid_len: device int32
 * [batch]; workspace: device, at least raya_postln_workspace_bytes.  Asynchronous on `stream`.
 * Every row of out is computed; rows at or beyond a sequence's valid length attend to nothing
 * (their attention output is zero). */
int raya_postln_layer_forward(const raya_postln_layer *layer, const int32_t *valid_len, const float *x, float *out,
                              void *workspace, uint64_t workspace_bytes, void *stream);

/* ---- Decision model (crates/raya-core, crates/raya-weights) ------------------------------
 *
 * Errors of this part are raya_core::Error (crates/raya-core/src/error.rs:5-33); the
 * message is the variant's Display text ("invalid config: `field`: reason",
 * "invalid input: …", "invalid weights file …" with its report, …). */
#define RAYA_ERR_CONFIG 5        /* Error::Config, Error::Io, Error::Json */
#define RAYA_ERR_UNIMPLEMENTED 6 /* Error::Unimplemented */
#define RAYA_ERR_INPUT 7         /* Error::Input */
#define RAYA_ERR_KERNEL 8        /* Error::Kernel: the attention kernel rejected the call */
#define RAYA_ERR_WEIGHTS 9       /* Error::Weights (LoadReport) */

typedef struct raya_model raya_model;

/* ModelConfig::from_dir (crates/raya-core/src/config/mod.rs:26-39) on
 * checkpoint_dir, then raya_weights::load (crates/raya-weights/src/store.rs:66-151)
 * of weights_path (NULL: checkpoint_dir/model.safetensors, as load_dir,
 * store.rs:234-239) against the parameter set the config implies
 * (mapping.rs:19-143).  F16/BF16 tensors are widened to fp32.  Host only: the
 * weights go to a device on the first forward call there, once. */
int raya_model_load(const char *checkpoint_dir, const char *weights_path, raya_model **out);
void raya_model_free(raya_model *model);

/* mapping::expected (crates/raya-weights/src/mapping.rs:19-40): the parameters,
 * in order, that a weights file for the config in checkpoint_dir must hold,
 * under raya-weights' names.  Writes min(capacity, count) entries; *count is
 * the full number. */
typedef struct raya_param_entry {
    char name[128];
    uint32_t ndim;
    uint64_t shape[4];
} raya_param_entry;

int raya_expected_params(const char *checkpoint_dir, raya_param_entry *out, uint64_t capacity,
                         uint64_t *count);

typedef struct raya_model_info {
    uint64_t hidden_size, intermediate_size, num_hidden_layers, num_attention_heads;
    uint64_t global_attn_every_n_layers, local_attention, vocab_size, max_position_embeddings;
    double global_rope_theta, local_rope_theta, norm_eps;
    uint64_t head_layers, head_heads, head_ffn, n_act;
    uint64_t param_floats; /* fp32 parameter storage, including per-tensor alignment */
} raya_model_info;

int raya_model_get_info(const raya_model *model, raya_model_info *info);

/* A batch of ForwardInput (crates/raya-core/src/model.rs:90-100), all host
 * arrays: sequence b has ids input_ids[b][0..seq), valid length valid_len[b]
 * (right padding), markers marker_pos[b][0..markers) with marker_mask, and
 * qtype[b].  A sequence with fewer markers pads with mask 0 entries (they act
 * as invalid markers, as in the reference).  local_override != 0 replaces the
 * local layers' Sliding(local_attention / 2) mask (encoder.rs:116-120) by
 * (local_mask_kind, local_mask_arg) — a throughput option, not the reference. */
typedef struct raya_forward_batch {
    uint64_t batch, seq, markers;
    const uint32_t *input_ids;
    const uint64_t *valid_len;
    const uint64_t *marker_pos;
    const uint8_t *marker_mask;
    const uint64_t *qtype;
    int32_t local_override;
    int32_t local_mask_kind;
    uint64_t local_mask_arg;
} raya_forward_batch;

/* ForwardOutput (model.rs:102-112) per sequence, host arrays (any may be NULL):
 * logits and probabilities [batch][markers], act_logits [batch][n_act],
 * features [batch][4], pooled [batch][hidden_size]. */
typedef struct raya_forward_output {
    float *logits, *probabilities, *act_logits, *features, *pooled;
} raya_forward_output;

/* Trace (crates/raya-core/src/trace.rs): called once per stage, in execution
 * order, under the golden fixtures' names (embedding_output, encoder_layer_00,
 * …, act_logits) with host data valid for the call.  Sequence-shaped stages
 * are [batch][seq][hidden] with zeros on padded rows. */
typedef void (*raya_trace_fn)(void *user, const char *name, const uint64_t *shape, uint32_t ndim,
                              const float *data);

/* Network::forward (model.rs:261-348) for every sequence of the batch in one
 * device pass: inputs are checked as Network::check does (model.rs:221-258)
 * before any device work; the valid tokens are packed and run through every
 * layer on the current device (weights uploaded there on first use); the
 * outputs are copied back and `stream` (hipStream_t, NULL = null stream) is
 * synchronised before returning.  trace may be NULL.  Calls on one model are
 * serialised. */
int raya_model_forward(raya_model *model, const raya_forward_batch *in, raya_forward_output *out,
                       raya_trace_fn trace, void *user, void *stream);

/* Stage timing, the forward's counterpart of Tiled::attend_with_stages
 * (crates/raya-kernels/src/tiled/mod.rs:61-126): with level 1,
 * raya_model_forward records a HIP event pair on its stream around the
 * embedding, each encoder layer, the final norm, each head layer and the
 * scorer + act head; with level 2 also around every kernel of an encoder layer
 * ("encoder_layer_03/qkv", "/attention", "/attn_out", "/mlp_norm",
 * "/mlp_in_geglu", "/mlp_out", "/attn_norm").  Level 0 (the default) records
 * nothing.  raya_model_stage_times returns the last forward's spans in order:
 * min(capacity, count) entries, *count the full number.  Spans that contain a
 * trace callback include its host copies. */
int raya_model_set_profiling(raya_model *model, int level);

typedef struct raya_stage_time {
    char name[48];
    double ms;
} raya_stage_time;

int raya_model_stage_times(raya_model *model, raya_stage_time *out, uint64_t capacity, uint64_t *count);

#ifdef __cplusplus
}
#endif

#endif
