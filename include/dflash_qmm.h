/*
 * dflash_qmm.h -- C ABI of the MI355X (gfx950) small-M affine-quantised matmul.
 *
 * This is the drop-in boundary for DFlashKit's SmallMQuantizedMatmul path.  In the
 * reference (paths relative to the reference repository root) the path sits behind MLX's
 * custom-kernel FFI and a Swift subclass of QuantizedLinear:
 *
 *   Sources/DFlashKit/SmallMQuantizedMatmul.swift:174-187  kernel objects built lazily
 *                                                          through MLXFast.metalKernel
 *   Sources/DFlashKit/SmallMQuantizedMatmul.swift:193-201  isEligible(_:)
 *   Sources/DFlashKit/SmallMQuantizedMatmul.swift:205-207  tiles(for:)
 *   Sources/DFlashKit/SmallMQuantizedMatmul.swift:210-224  apply(x:weight:scales:biases:...)
 *   Sources/DFlashKit/SmallMQuantizedMatmul.swift:234-293  SmallMQuantizedLinear
 *   Sources/DFlashKit/SmallMQuantizedMatmul.swift:303-317  enableSmallMQuantizedMatmul(in:)
 *
 * Each declaration below names the reference item it replaces.  Conventions:
 *   - every function returns a dfq_status (0 = DFQ_OK) unless stated; nothing aborts or
 *     throws across the ABI; dfq_last_error() returns a thread-local message;
 *   - all device buffers are caller-owned (no allocation on the matmul path);
 *   - streams are hipStream_t passed as void* (NULL = the default stream);
 *   - weights are consumed in MLX's layout, in place: w uint32 [N][K*bits/32] with element 0
 *     in the low bits, scales and biases [N][K/group_size];
 *   - calls are re-entrant per stream; concurrent calls that share one workspace race.
 */
#ifndef DFLASH_QMM_H
#define DFLASH_QMM_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define DFQ_ABI_VERSION 1

typedef enum dfq_status {
    DFQ_OK = 0,
    DFQ_ERR_INVALID_ARGUMENT = 1, /* null pointer, negative size, misaligned buffer      */
    DFQ_ERR_UNSUPPORTED = 2,      /* shape / format outside what the called path handles */
    DFQ_ERR_WORKSPACE = 3,        /* workspace missing or smaller than required          */
    DFQ_ERR_HIP = 4,              /* a HIP runtime call failed                           */
    DFQ_ERR_NO_DEVICE = 5,        /* no gfx950 device, or code object failed to load     */
    DFQ_ERR_STATE = 6             /* call out of order (e.g. graph_end without begin)    */
} dfq_status;

typedef enum dfq_dtype { DFQ_BF16 = 0, DFQ_F16 = 1, DFQ_F32 = 2 } dfq_dtype;

typedef struct dfq_ctx dfq_ctx;
typedef struct dfq_graph dfq_graph;

/* ---- the eligibility window (SmallMQuantizedMatmul.swift:29-49) -------------------- */
/* :32 minimumRows, "a constant of (chip x MLX version)" (:29-31): the fewest rows for which
 * the fast kernel clearly beats the stock path the layer falls through to, MLX's GEMV on the
 * reference's Apple GPU (6 there).  On MI355X the stock path is dfq_qmm_fallback's GEMV;
 * measured against it (us, stock / fast kernel), one row is a draw -- 4096 x 4096:
 * 6.3 / 7.4, 5120 x 5120: 8.2 / 9.7, 17408 x 5120: 15.5 / 15.3, 5120 x 17408: 16.0 / 15.9,
 * 151936 x 5120: 90.8 / 78.8 -- and two rows are the first clear win (17408 x 5120:
 * 18.3 / 15.0, 5120 x 17408: 19.9 / 15.7, 151936 x 5120: 100.7 / 79.3). */
#define DFQ_MINIMUM_ROWS 2
#define DFQ_MAXIMUM_ROWS 16              /* :36 maximumRows                              */
#define DFQ_ROWS_PER_TILE 8              /* :39 rowsPerTile (also read by the generator's
                                            width snapping, DFlashSpeculativeGenerator.swift
                                            :136-142, 325-326)                           */
#define DFQ_MINIMUM_OUTPUT_FEATURES 4096 /* :41 minimumOutputFeatures                    */
#define DFQ_INPUT_FEATURE_MULTIPLE 512   /* :45 inputFeatureMultiple                     */
#define DFQ_REQUIRED_GROUP_SIZE 64       /* :47 requiredGroupSize                        */

/* ---- context ---------------------------------------------------------------------- */

/* Loads the gfx950 code object (hipModuleLoadData) and resolves every kernel.
 * Replaces the lazily built kernel table, SmallMQuantizedMatmul.swift:169-187. */
dfq_status dfq_init(int device, dfq_ctx** out);
dfq_status dfq_destroy(dfq_ctx* ctx);
const char* dfq_last_error(void);
const char* dfq_status_string(dfq_status s);
int dfq_abi_version(void);
/* Number of compute units the work split is sized for. */
int dfq_num_cus(const dfq_ctx* ctx);

/* ---- device memory and streams (so a host without HIP headers can drive the path) -- */
dfq_status dfq_malloc(dfq_ctx* ctx, size_t bytes, void** out);
dfq_status dfq_free(dfq_ctx* ctx, void* ptr);
dfq_status dfq_memcpy_h2d(dfq_ctx* ctx, void* dst, const void* src, size_t bytes, void* stream);
dfq_status dfq_memcpy_d2h(dfq_ctx* ctx, void* dst, const void* src, size_t bytes, void* stream);
dfq_status dfq_stream_create(dfq_ctx* ctx, void** stream);
dfq_status dfq_stream_destroy(dfq_ctx* ctx, void* stream);
dfq_status dfq_stream_sync(dfq_ctx* ctx, void* stream);

/* ---- the eligibility gate ------------------------------------------------------------ */

/* Static half of the gate: mode == affine, biases present, bits in {4, 8},
 * group_size == 64, N >= 4096, K % 512 == 0.  Returns 1 / 0.
 * Replaces SmallMQuantizedMatmul.isEligible(_:), SmallMQuantizedMatmul.swift:193-201. */
int dfq_is_eligible(int out_features, int in_features, int bits, int group_size,
                    int mode_affine, int has_biases);

/* MMA tiles of 8 rows a pass of `rows` rows pays for: 1 up to 8, else 2.
 * Replaces SmallMQuantizedMatmul.tiles(for:), SmallMQuantizedMatmul.swift:205-207. */
int dfq_tiles_for(int rows);

/* Whether dfq_qmm's kernels handle this problem (wider than the reference gate: any
 * M in 1..16, N >= 1, group 32/64/128, bits 4/8, bf16 or fp16 throughout, K a multiple
 * of the kernel's super-step).  9..16 rows run in one launch with two row tiles per
 * weight tile when K is a multiple of 8 groups, else as two launches of up to 8 rows.
 * Returns 1 / 0. */
int dfq_qmm_supported(const dfq_ctx* ctx, int M, int N, int K, int bits, int group_size,
                      dfq_dtype x_dtype, dfq_dtype sb_dtype, dfq_dtype y_dtype);

/* ---- the matmul ------------------------------------------------------------------- */

/* Workspace dfq_qmm needs for this shape (0 if none).  The workspace must be zero-filled
 * once before its first use (dfq_workspace_clear); every call leaves all of it zero again,
 * so one workspace serves calls of any shape in stream order. */
dfq_status dfq_qmm_workspace_bytes(dfq_ctx* ctx, int M, int N, int K, int bits,
                                   int group_size, size_t* bytes);
dfq_status dfq_workspace_clear(dfq_ctx* ctx, void* workspace, size_t bytes, void* stream);

/* y[M,N] = x[M,K] . dequant(w)[N,K]^T (+ linear_bias[N]) on the fast kernel.
 * x, scales, biases, linear_bias and y share one dtype (bf16 or fp16); y dtype = x dtype.
 * Asynchronous on `stream`; allocates nothing.
 * Replaces SmallMQuantizedMatmul.apply(...) (SmallMQuantizedMatmul.swift:210-224) and the
 * MLXFastKernel call it makes (:217-223); the optional linear bias is the `y + bias` of
 * SmallMQuantizedLinear.callAsFunction (:288-290), fused before the final rounding. */
dfq_status dfq_qmm(dfq_ctx* ctx, const void* x, const uint32_t* w, const void* scales,
                   const void* biases, const void* linear_bias, void* y, int M, int N, int K,
                   int bits, int group_size, dfq_dtype x_dtype, dfq_dtype sb_dtype,
                   dfq_dtype y_dtype, void* workspace, size_t workspace_bytes, void* stream);

/* dfq_qmm with no workspace argument, for callers that cannot allocate device memory (code
 * under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).  No
 * counterpart in the reference, where MLX allocates every output and scratch itself.
 * The workspace is a fixed array of DFQ_SCRATCH_MAX_BYTES per GPU inside the library, taken
 * at dfq_init and held until the process ends; this call allocates nothing (no hipMalloc,
 * hipFree or host allocation) and returns DFQ_ERR_WORKSPACE for a shape whose workspace
 * (dfq_qmm_workspace_bytes) is larger.  Every call on one GPU shares that array: calls that
 * overlap on one GPU (other streams, other threads, other contexts) race, so serialise
 * them.  Each call leaves the array zero, as dfq_qmm leaves its workspace; a call that fails
 * after queueing a launch queues a clear of the bytes its shape uses.  The work split of a
 * shape is planned once per context: shapes dfq_qmm has not met go to a fixed table of 64
 * entries made with the context.  Same arguments, results and errors as dfq_qmm otherwise
 * (bit-identical outputs). */
#define DFQ_SCRATCH_MAX_BYTES ((size_t)64 << 20)
dfq_status dfq_qmm_noalloc(dfq_ctx* ctx, const void* x, const uint32_t* w, const void* scales,
                           const void* biases, const void* linear_bias, void* y, int M, int N,
                           int K, int bits, int group_size, dfq_dtype x_dtype,
                           dfq_dtype sb_dtype, dfq_dtype y_dtype, void* stream);

/* The MLP's fused gate|up projection with its SiLU-mul epilogue: h[M][H] = silu(x . Wg^T) *
 * (x . Wu^T), over one weight whose gate and up rows are interleaved in blocks of 8 (rows
 * 16b..16b+7 = gate rows 8b.., rows 16b+8.. = up rows 8b..; dfq_interleave_gate_up builds it,
 * and the scales, biases and linear bias alike).  g and u are rounded to the dtype before
 * silu, exactly as dfq_silu_mul applied to the stored gate|up output, so h is bit-identical
 * to that pair of calls on the interleaved weight.  H % 8 == 0; the workspace is
 * dfq_qmm_workspace_bytes(M, 2*H, K, ...).  The fused form of the MLP activation of the
 * target layers (the SiLU-gated MLP of DFlashDecoderLayer.swift:26) around the swapped
 * gate and up projections. */
dfq_status dfq_qmm_silu_gate_up(dfq_ctx* ctx, const void* x, const uint32_t* w_gu,
                                const void* scales_gu, const void* biases_gu,
                                const void* linear_bias_gu, void* h, int M, int H, int K,
                                int bits, int group_size, dfq_dtype dtype, void* workspace,
                                size_t workspace_bytes, void* stream);
/* out[2H rows] = gate and up rows (row_bytes each) interleaved in blocks of 8, on `stream`;
 * for the weight (row_bytes = K*bits/8), scales and biases (K/group_size*2) and linear bias
 * (2). */
dfq_status dfq_interleave_gate_up(dfq_ctx* ctx, const void* gate, const void* up, void* out,
                                  int H, size_t row_bytes, void* stream);

/* The stock path: any M >= 1, bits 2/4/8, any group size dividing K; x and scales may
 * differ in dtype (y dtype follows MLX promotion: equal -> same, else fp32).  Stands in for
 * the stock op MLX falls back to, QuantizedLinear.callAsFunction -> quantizedMatmul (reached
 * at SmallMQuantizedMatmul.swift:265), which runs a GEMV for few rows.  Where x, scales and y
 * share bf16 or fp16, bits are 4 or 8, the group 32, 64 or 128 and 4 rows of x fit in LDS, it
 * runs as that GEMV, one launch per 4 rows (each weight row read once a launch); otherwise
 * one wave per output element, re-reading W for every row.  No workspace; asynchronous on
 * `stream`. */
dfq_status dfq_qmm_fallback(dfq_ctx* ctx, const void* x, const uint32_t* w, const void* scales,
                            const void* biases, const void* linear_bias, void* y, int M, int N,
                            int K, int bits, int group_size, dfq_dtype x_dtype,
                            dfq_dtype sb_dtype, dfq_dtype y_dtype, void* stream);

/* ---- graph capture of a layer's matmul chain ------------------------------------------ */
/* Stream capture of whatever the caller enqueues on `stream` between begin and end
 * (typically the q/k/v/o/gate/up/down dfq_qmm calls of one layer), instantiated once and
 * replayed with dfq_graph_launch.  No counterpart in the reference (MLX builds a lazy graph
 * per forward, DFlashSpeculativeGenerator.swift:389-398); it is the HIP-native way to issue
 * one verify-pass layer. */
dfq_status dfq_graph_begin(dfq_ctx* ctx, void* stream);
dfq_status dfq_graph_end(dfq_ctx* ctx, void* stream, dfq_graph** out);
dfq_status dfq_graph_launch(dfq_graph* graph, void* stream);
dfq_status dfq_graph_destroy(dfq_graph* graph);
/* One graph that runs the n captured graphs parts[0..n-1] one after the other (each as a
 * child-graph node depending on the previous one), instantiated once: the verify forward's
 * per-layer graphs launched as one.  The parts are copied in; they stay valid and owned by
 * the caller.  Launched graphs follow each other with a gap of several microseconds on
 * MI355X (the runtime's graph launch), the kernels of one graph do not: 64 layer graphs
 * composed run as fast as the forward captured as one graph.  No counterpart in the
 * reference (DFlashSpeculativeGenerator.swift:389-398 issues one lazy MLX graph per
 * forward). */
dfq_status dfq_graph_compose(dfq_ctx* ctx, dfq_graph* const* parts, int n, dfq_graph** out);

/* ---- the packed layout ---------------------------------------------------------------- */
/* A weight prepared once at load for the fast kernel: the MLX arrays (codes, scales, biases)
 * of 16 output rows by 8 quantisation groups, the unit one lane group of the kernel loads,
 * stored as one contiguous piece -- the codes as the kernel's lanes load them (1 KB per load
 * instruction), then the rows' scales and biases (512 bytes) -- in tile-major order, rows past
 * N zero.  The kernel then reads each unit as whole cache lines instead of 16 rows' pieces of
 * the weight and 32 pieces of the two 16-bit arrays: on MI355X the kernel's own loads of the
 * 17408 x 5120 4-bit weight take 10.6 us packed against 11.4 us in the MLX layout, and of the
 * 151936 x 5120 LM head 72 us against 82-85 us.  Results are bit-identical to the MLX layout's
 * (the same values reach the same registers).  No counterpart in the reference, which reads
 * MLX's arrays in place (SmallMQuantizedMatmul.swift:127-129, 140); the packed copy holds the
 * same bytes as those arrays (rounded up to whole tiles of 16 rows), so a loader that packs
 * and drops them uses no extra memory.
 *
 * dfq_packed_bytes: its size for an N x K weight (K a multiple of 8 groups; 4 or 8 bits;
 * groups of 32, 64 or 128).  dfq_pack_weights: builds it on `stream` from 16-byte aligned MLX
 * arrays into a 256-byte aligned buffer.  dfq_qmm_packed, dfq_qmm_silu_gate_up_packed and
 * dfq_qmm_argmax_accept_packed: dfq_qmm, dfq_qmm_silu_gate_up and dfq_qmm_argmax_accept over
 * it (one dtype for x, scales, biases and the outputs; the same workspaces). */
dfq_status dfq_packed_bytes(int N, int K, int bits, int group_size, size_t* bytes);
dfq_status dfq_pack_weights(dfq_ctx* ctx, const uint32_t* w, const void* scales,
                            const void* biases, int N, int K, int bits, int group_size,
                            void* packed, void* stream);
dfq_status dfq_qmm_packed(dfq_ctx* ctx, const void* x, const void* packed,
                          const void* linear_bias, void* y, int M, int N, int K, int bits,
                          int group_size, dfq_dtype dtype, void* workspace,
                          size_t workspace_bytes, void* stream);
dfq_status dfq_qmm_silu_gate_up_packed(dfq_ctx* ctx, const void* x, const void* packed_gu,
                                       const void* linear_bias_gu, void* h, int M, int H, int K,
                                       int bits, int group_size, dfq_dtype dtype,
                                       void* workspace, size_t workspace_bytes, void* stream);
dfq_status dfq_qmm_argmax_accept_packed(dfq_ctx* ctx, const void* x, const void* packed,
                                        const void* linear_bias, void* logits, int M, int V,
                                        int K, int bits, int group_size, dfq_dtype dtype,
                                        const int32_t* proposals, int32_t* tokens,
                                        int32_t* accepted, void* workspace,
                                        size_t workspace_bytes, void* stream);

/* h[m][n] = silu(gu[m][n]) * gu[m][N + n] for the fused gate||up projection's output
 * gu[M][2N] (row pitch 2N elements): the activation between gate||up and down in a layer
 * chain.  bf16 or fp16, computed in fp32 (silu(g) = g / (1 + e^-g)) and rounded once.  No
 * counterpart on the reference's path: MLX runs SiLU and the product as its own ops in the
 * model's MLP, around the swapped projections (SmallMQuantizedMatmul.swift:303-317). */
dfq_status dfq_silu_mul(dfq_ctx* ctx, const void* gu, void* h, int M, int N, dfq_dtype dtype,
                        void* stream);

/* ---- greedy accept of a verify pass ---------------------------------------------------- */
/* tokens[m] = argmax over V of logits[m][*] (first index among equal maxima, NaN skipped;
 * -1 for a row with no number) for the M = 1 + drafts verify positions, and
 * *accepted = the leading run of proposals[i] == tokens[i], i < M - 1 (the sum of the
 * cumulative product of the matches).  On the device: only these M + 1 ints need to reach
 * the host.  proposals, tokens or accepted may be NULL (no proposals: accepted = 0).
 * Replaces acceptedPrefix(targetLogits:proposals:) (DFlashSpeculativeGenerator.swift:555-571,
 * argMax / == / cumprod / sum at :562-564).  The workspace (dfq_argmax_accept_workspace_bytes,
 * 8-byte aligned) must be zero before the first call (dfq_workspace_clear); every call
 * leaves it zero. */
dfq_status dfq_argmax_accept_workspace_bytes(int M, size_t* bytes);
dfq_status dfq_argmax_accept(dfq_ctx* ctx, const void* logits, int M, int V, dfq_dtype dtype,
                             const int32_t* proposals, int32_t* tokens, int32_t* accepted,
                             void* workspace, size_t workspace_bytes, void* stream);

/* The LM head fused with the greedy accept: logits[M][V] = x . dequant(w)^T (+ linear bias)
 * on the fast kernel, and from them, as dfq_argmax_accept computes them, tokens[m] (the first
 * index of each row's largest logit, NaN skipped, -1 for a row with no number) and *accepted
 * (the leading run of proposals[i] == tokens[i], i < M-1).  Every logit is folded into its
 * row's key where the kernel finishes it, and the last workgroup decodes the keys: the
 * logits need not go to memory and no second kernel reads them back.  logits may be NULL
 * (then nothing of them is written).  Results are identical to dfq_qmm followed by
 * dfq_argmax_accept on its output.  Shapes whose split needs the second pass (dfq_qmm's
 * reduce splits), or whose K is not a multiple of 8 groups, run as exactly that pair of
 * calls, with the logits in `logits` or, when it is NULL, in the workspace's tail.  dtype is
 * that of x, scales, biases and the logits.  The
 * workspace (dfq_qmm_argmax_accept_workspace_bytes, 256-byte aligned) must be zero before
 * the first call (dfq_workspace_clear); every call leaves it zero again, except the logits
 * tail of that two-call form, which only ever holds logits and needs no clearing.
 * Replaces the lm_head projection and acceptedPrefix(targetLogits:proposals:) of a verify
 * round (DFlashSpeculativeGenerator.swift:389-398, 555-571; argMax / == / cumprod / sum at
 * :562-564): only M tokens and one count leave the device. */
dfq_status dfq_qmm_argmax_accept_workspace_bytes(dfq_ctx* ctx, int M, int V, int K, int bits,
                                                 int group_size, size_t* bytes);
dfq_status dfq_qmm_argmax_accept(dfq_ctx* ctx, const void* x, const uint32_t* w,
                                 const void* scales, const void* biases,
                                 const void* linear_bias, void* logits, int M, int V, int K,
                                 int bits, int group_size, dfq_dtype dtype,
                                 const int32_t* proposals, int32_t* tokens, int32_t* accepted,
                                 void* workspace, size_t workspace_bytes, void* stream);

/* ---- the drop-in layer (SmallMQuantizedMatmul.swift:227-317) -------------------------- */

typedef struct dfq_linear dfq_linear;
typedef struct dfq_model dfq_model;

/* A quantised linear layer over caller-owned device arrays (MLX's QuantizedLinear fields:
 * weight, scales, biases, bias, groupSize, bits, mode).  Nothing is copied. */
typedef struct dfq_linear_desc {
    const uint32_t* weight;   /* [out][in*bits/32]                                   */
    const void* scales;       /* [out][in/group_size]                                */
    const void* biases;       /* [out][in/group_size], NULL if the mode has none     */
    const void* bias;         /* [out] linear bias or NULL                           */
    int out_features, in_features, bits, group_size;
    int mode_affine;          /* 1 = MLX .affine                                     */
    dfq_dtype dtype;          /* dtype of scales / biases / bias                     */
} dfq_linear_desc;

/* A stock QuantizedLinear: every call goes to the generic path.  ctx may be NULL for a
 * layer that is only inspected or swapped (its forward then returns DFQ_ERR_STATE). */
dfq_status dfq_linear_create(dfq_ctx* ctx, const dfq_linear_desc* desc, dfq_linear** out);
/* SmallMQuantizedLinear(other): wraps `other`, sharing its arrays (:243-252). */
dfq_status dfq_small_m_linear_create(dfq_linear* other, dfq_linear** out);
dfq_status dfq_linear_destroy(dfq_linear* lin);
/* 1 if `lin` is a SmallMQuantizedLinear. */
int dfq_linear_is_small_m(const dfq_linear* lin);
/* Gives a SmallMQuantizedLinear a copy of its weight in the packed layout (dfq_pack_weights),
 * which its fast-kernel calls then read (bit-identical results); the stock path keeps reading
 * the MLX arrays, so the layer holds its weight twice.  The copy belongs to the layer (freed
 * with it and with every handle sharing it) and is built on `stream`; returns when done.
 * DFQ_ERR_UNSUPPORTED for a layer whose calls never take the fast kernel (not eligible, not
 * bf16) or whose format has no packed form (the layer is left as it was);
 * DFQ_ERR_INVALID_ARGUMENT for a stock layer.  A second call does nothing.  No counterpart
 * in the reference, which reads MLX's arrays in place (SmallMQuantizedMatmul.swift:245-248). */
dfq_status dfq_small_m_linear_pack(dfq_linear* lin, void* stream);
/* The layer's weight in the packed layout, or NULL if it has none. */
const void* dfq_linear_packed(const dfq_linear* lin);
/* The dtype callAsFunction returns for input dtype x_dtype. */
dfq_dtype dfq_linear_output_dtype(const dfq_linear* lin, dfq_dtype x_dtype);
/* callAsFunction (:254-292): y[rows][out] for x[rows][in]; rows = product of the leading
 * dimensions.  A SmallMQuantizedLinear takes the fast kernel when it is eligible,
 * DFQ_MINIMUM_ROWS <= rows <= DFQ_MAXIMUM_ROWS and x is bf16, and falls through to the
 * stock path otherwise; *took_kernel (may be NULL) reports which. */
dfq_status dfq_linear_forward(dfq_linear* lin, const void* x, dfq_dtype x_dtype, int rows,
                              void* y, void* workspace, size_t workspace_bytes, void* stream,
                              int* took_kernel);
/* Workspace the layer's forward needs at `rows` rows. */
dfq_status dfq_linear_workspace_bytes(dfq_linear* lin, int rows, size_t* bytes);

/* A module tree reduced to what the swap needs: named leaf layers. */
dfq_status dfq_model_create(dfq_model** out);
dfq_status dfq_model_destroy(dfq_model* model);
/* Adds (or replaces) the leaf at `path`; the model takes ownership of `lin`.  A handle the
 * model already owns (set at another path, as for a tied layer, or returned by
 * dfq_model_leaf) may be set again: it stays owned once and is freed once. */
dfq_status dfq_model_set_leaf(dfq_model* model, const char* path, dfq_linear* lin);
/* The leaf at `path` (NULL if none) as a borrowed handle: never pass it to
 * dfq_linear_destroy.  It stays valid until dfq_model_destroy, also after the leaf is
 * swapped or replaced (it then still describes the layer it named). */
dfq_linear* dfq_model_leaf(dfq_model* model, const char* path);
int dfq_model_leaf_count(const dfq_model* model);
/* Swaps every eligible stock leaf for a SmallMQuantizedLinear; returns how many were
 * swapped (idempotent: already-swapped leaves are skipped), or -1 on error.
 * Replaces enableSmallMQuantizedMatmul(in:), SmallMQuantizedMatmul.swift:303-317. */
int dfq_enable_small_m_quantized_matmul(dfq_model* model);

/* ---- MLX quantised checkpoints (safetensors) ------------------------------------------
 * The on-disk format the fast kernel consumes, loaded as it is: for each quantised layer P,
 * P.weight (U32 [out][in*bits/32]), P.scales and P.biases ([out][in/group_size], BF16 / F16
 * / F32) and optionally the linear bias P.bias ([out]).  A layer is quantised when P.scales
 * and P.weight exist; its bits and group size come from config.json's "quantization" object
 * (top-level group_size / bits, overridden by an entry keyed by P; an entry of false turns
 * the layer off), or from dfq_checkpoint_set_quantization.  Replaces, for the layers this path
 * serves, the quantised-weight half of loadModel (mlx-swift-lm; reached at
 * Sources/dflash-bench/main.swift:26) that fills the QuantizedLinear fields SmallMQuantized-
 * Linear shares (SmallMQuantizedMatmul.swift:245-248). */

typedef struct dfq_checkpoint dfq_checkpoint;

typedef enum dfq_st_dtype {
    DFQ_ST_BOOL = 0, DFQ_ST_U8, DFQ_ST_I8, DFQ_ST_I16, DFQ_ST_U16, DFQ_ST_F16, DFQ_ST_BF16,
    DFQ_ST_I32, DFQ_ST_U32, DFQ_ST_F32, DFQ_ST_I64, DFQ_ST_U64, DFQ_ST_F64, DFQ_ST_F8_E5M2,
    DFQ_ST_F8_E4M3
} dfq_st_dtype;

typedef struct dfq_tensor_info {
    const char* name;     /* valid until dfq_checkpoint_close                           */
    dfq_st_dtype dtype;
    int ndim;
    int64_t shape[8];
    uint64_t nbytes;
    int shard;            /* index of the file holding it (sorted file names)           */
    uint64_t offset;      /* absolute byte offset of its data in that file              */
} dfq_tensor_info;

typedef struct dfq_layer_info {
    const char* prefix;   /* P; valid until dfq_checkpoint_close                        */
    int out_features, in_features, bits, group_size;
    int has_biases, has_bias;
    dfq_dtype dtype;      /* of scales / biases / bias                                  */
    int valid;            /* 1: the tensors agree with bits / group size and can load   */
    const char* problem;  /* why not ("" when valid); changes with set_quantization     */
} dfq_layer_info;

/* Opens a .safetensors file, or a directory of model*.safetensors shards (every
 * *.safetensors when none is so named) with an optional config.json, and checks every
 * header: dtype known, shape matching the byte range, ranges inside the file, no name in
 * two shards.  Reads no tensor data. */
dfq_status dfq_checkpoint_open(const char* path, dfq_checkpoint** out);
/* Closes the files and frees the device memory of every dfq_checkpoint_load_model call:
 * destroy models loaded from it first. */
dfq_status dfq_checkpoint_close(dfq_checkpoint* ck);
/* The header's __metadata__ "format" ("mlx" for MLX checkpoints; "" if none). */
const char* dfq_checkpoint_format(const dfq_checkpoint* ck);
int dfq_checkpoint_tensor_count(const dfq_checkpoint* ck);
dfq_status dfq_checkpoint_tensor(const dfq_checkpoint* ck, int index, dfq_tensor_info* out);
dfq_status dfq_checkpoint_find(const dfq_checkpoint* ck, const char* name, dfq_tensor_info* out);
/* A tensor's bytes into host memory, as stored. */
dfq_status dfq_checkpoint_read(const dfq_checkpoint* ck, const char* name, void* dst,
                               size_t bytes);
/* A tensor's bytes into caller-owned device memory, as stored (returns when done). */
dfq_status dfq_checkpoint_upload(dfq_ctx* ctx, dfq_checkpoint* ck, const char* name, void* dst,
                                 size_t bytes, void* stream);
/* Bits and group size of layer `prefix`, or of every layer without its own (prefix NULL). */
dfq_status dfq_checkpoint_set_quantization(dfq_checkpoint* ck, const char* prefix, int bits,
                                           int group_size);
/* The quantised layers, sorted by prefix. */
int dfq_checkpoint_layer_count(const dfq_checkpoint* ck);
dfq_status dfq_checkpoint_layer(const dfq_checkpoint* ck, int index, dfq_layer_info* out);
/* Loads every quantised layer for which want(prefix, user) is non-zero (want NULL: all)
 * into one device allocation, in the file layout, and adds each to `model` as a stock
 * QuantizedLinear leaf named by its prefix (dfq_enable_small_m_quantized_matmul then swaps
 * the eligible ones).  Fails before allocating if a chosen layer is not valid.  Files are
 * read in order through pinned staging buffers; returns when the data is on the device.
 * *loaded (may be NULL) gets the number of layers added. */
dfq_status dfq_checkpoint_load_model(dfq_ctx* ctx, dfq_checkpoint* ck, dfq_model* model,
                                     int (*want)(const char* prefix, void* user), void* user,
                                     void* stream, int* loaded);
/* dfq_checkpoint_load_model with every chosen layer that the packed layout serves (an affine
 * layer with biases, 4 or 8 bits, bf16 or fp16 scales, K a multiple of 8 groups, a fast-kernel
 * split at 1..16 rows) written into the allocation in that layout instead of MLX's: the same
 * bytes (rows rounded up to 16), through a device staging buffer of up to 1 GiB (or the
 * largest such layer) that is freed before it returns.  Other layers load as stored.  A
 * packed layer has no MLX arrays (dfq_linear_describe gives NULL weight, scales and biases;
 * dfq_linear_packed gives its weight): its stock path is the fast kernel over the packed
 * layout, 16 rows a launch, with x in the dtype of its scales; swapped, it takes the window
 * like any SmallMQuantizedLinear.  No counterpart in the reference, whose loader fills MLX
 * arrays (mlx-swift-lm loadModel, reached at Sources/dflash-bench/main.swift:26). */
dfq_status dfq_checkpoint_load_model_packed(dfq_ctx* ctx, dfq_checkpoint* ck, dfq_model* model,
                                            int (*want)(const char* prefix, void* user),
                                            void* user, void* stream, int* loaded);
/* The arrays and shape of a layer (for layers the caller did not create itself). */
dfq_status dfq_linear_describe(const dfq_linear* lin, dfq_linear_desc* out);

#ifdef __cplusplus
}
#endif

#endif /* DFLASH_QMM_H */
