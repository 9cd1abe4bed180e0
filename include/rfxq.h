/*
 * rfxq -- MI355X (gfx950) GGUF quantized-matmul library: the C ABI.
 *
 * Drop-in for the quantized-matmul path of the reference engine's Rust `Model`
 * (src/model/kernels.rs, src/model/dense.rs, src/moe.rs). Every entry point
 * takes plain device pointers, sizes and a hipStream_t, writes every element of
 * its outputs, launches on that stream only and adds no host synchronisation
 * (except rfxq_moe_ffn_grouped, whose routing needs the host logits, as the
 * reference's does). Weights are raw GGUF blocks, row-major [out][in/QK],
 * never repacked.
 *
 * Errors: every int-returning call returns 0 (RFXQ_OK) or an error code; the
 * message is then available from rfxq_last_error() on the calling thread
 * (pattern of src/ffi.rs:112-127 reflex_last_error / reflex_last_error_code).
 * Codes reuse the reference's ReflexErrorCode values (include/reflex_engine.h:55-72).
 */
#ifndef RFXQ_H
#define RFXQ_H

#include <stdint.h>
#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

#define RFXQ_OK 0
#define RFXQ_ERR_GGUF 1           /* type without a kernel here (ReflexError::Gguf) */
#define RFXQ_ERR_GPU 3            /* a HIP call failed (ReflexError::Cuda) */
#define RFXQ_ERR_OUT_OF_MEMORY 5  /* device allocation failed */
#define RFXQ_ERR_IO 10            /* file open / map failed (ReflexError::Io) */
#define RFXQ_ERR_INVALID_INPUT 11 /* bad argument (null pointer, k out of range, ...) */
#define RFXQ_ERR_OTHER 12         /* shape / alignment precondition (ReflexError::Other) */

/* ggml type ids, as in GGUF files (src/gguf.rs:124-152). */
#define RFXQ_TYPE_F32 0
#define RFXQ_TYPE_F16 1
#define RFXQ_TYPE_Q8_0 8
#define RFXQ_TYPE_Q8_1 9
#define RFXQ_TYPE_Q4_K 12
#define RFXQ_TYPE_Q6_K 14

/*
 * A quantized-resident weight: `Weight { data: WeightData::Quant { ty, arena,
 * offset, len }, shape }` (src/model/loading.rs:139-165). `data` is the device
 * address arena + offset; shape is [in_features, out_features] or, for a
 * stacked per-expert tensor, [in_features, out_features, expert_count].
 * Alignment preconditions (src/kernels_cuda/gemv_q4k.cu:60-63): Q4_K data is
 * 16-byte aligned; Q6_K and Q8_0 data are 2-byte aligned.
 */
typedef struct rfxq_weight {
    uint32_t ggml_type;
    uint32_t in_features;   /* K */
    uint32_t out_features;  /* N */
    uint32_t expert_count;  /* 0 for a 2-D weight */
    const void* data;       /* device pointer to the raw blocks */
    uint64_t len;           /* bytes */
} rfxq_weight;

/* One GEMV of a fused launch: y[N] = W . x[K]. */
typedef struct rfxq_gemv_item {
    const float* x;
    const rfxq_weight* w;
    float* y;
} rfxq_gemv_item;

typedef struct rfxq_gemv_plan rfxq_gemv_plan;

/* ---- errors / setup ---------------------------------------------------- */

/* Message of this thread's last failing call, or NULL (src/ffi.rs:112-127). */
const char* rfxq_last_error(void);
/* Code of this thread's last failing call, or RFXQ_OK. */
int rfxq_last_error_code(void);
/* Load the embedded gfx950 code object on `device` now (otherwise on first use),
 * like the reference's lazy module load (src/aot.rs:136-160, kernels.rs:948-959). */
int rfxq_init(int device);
/* ---- options and the GEMM path policy ----------------------------------- */

/* The prefill path's switches. They are read from the environment once, on
 * first use, with the reference's strict parsing (QuantMmaKernels::from_env,
 * src/model/kernels.rs:747-802; quant_fused_max_rows, :4180-4194). An
 * invalid value makes every call that needs the options fail with
 * RFXQ_ERR_INVALID_INPUT and the reference's message ("REFLEX_QUANT_MMA must be
 * 1 (the default) or 0, got \"2\""); like the reference, an unparsable
 * REFLEX_QUANT_FUSED_MAX_ROWS keeps its default. */
typedef struct rfxq_options {
    int32_t quant_mma;           /* REFLEX_QUANT_MMA: 1 (default) MMA prefill, 0: every row as a GEMV */
    uint32_t quant_mma_splits;   /* REFLEX_QUANT_MMA_SPLITS: 0 = chosen per GEMM, else the split-K count */
    uint32_t quant_mma_max_rows; /* REFLEX_QUANT_MMA_MAX_ROWS: 0 = no cap; above it rows run as GEMVs */
    uint32_t quant_mma_tile;     /* REFLEX_QUANT_MMA_TILE: 0 = chosen, 64 or 128 rows (int8 kernels) */
    int32_t mmq_f16;             /* REFLEX_MMQ_F16: 1 (default) f16-activation kernels, 0: int8 (Q8_1) kernels */
    uint32_t fused_max_rows;     /* REFLEX_QUANT_FUSED_MAX_ROWS (default 16): up to this many rows run as GEMVs */
} rfxq_options;

/* The current options (the environment's, or the last rfxq_set_options). */
int rfxq_get_options(rfxq_options* out);
/* Replace the options for later calls, like the reference's test setters
 * (QuantMmaKernels::set_enabled / set_splits, kernels.rs:804-830). Calls
 * already running keep the options they started with. Rejects
 * (RFXQ_ERR_INVALID_INPUT) quant_mma or mmq_f16 other than 0/1 and a tile
 * other than 0, 64 or 128. */
int rfxq_set_options(const rfxq_options* options);

#define RFXQ_PATH_GEMV_ROWS 0  /* one decode GEMV per row (f16 activations) */
#define RFXQ_PATH_MMQ_INT8 1   /* int8 MMQ kernels on Q8_1 activations */
#define RFXQ_PATH_MMQ_F16 2    /* f16-activation MMQ kernels (Q4_K, Q6_K) */

/* How rfxq_gemm runs a GEMM: the path, the workgroup tile and the split-K
 * (splits ranges of sb_per_split super-blocks); tile and splits are 0/1 on the
 * GEMV path. Counterpart of quant_mma_splits / quant_mma_block_rows /
 * quant_mma_max_rows (kernels.rs:628-713) and the fused-GEMV crossover
 * (:2144-2169), re-derived for MI355X; `compute_units` as the device reports. */
typedef struct rfxq_gemm_policy {
    uint32_t path;
    uint32_t tile_m, tile_n;
    uint32_t splits, sb_per_split;
} rfxq_gemm_policy;
int rfxq_gemm_policy_for(uint32_t ggml_type, uint32_t in_features, uint32_t out_features, uint32_t rows,
                         uint32_t compute_units, rfxq_gemm_policy* out);

/* (elements per block, bytes per block) of a ggml type (src/gguf.rs:366-400). */
int rfxq_block_dims(uint32_t ggml_type, uint32_t* block_elems, uint32_t* block_bytes);

/* ---- dequantization ------------------------------------------------------ */

/* Raw Q4_K / Q6_K / Q8_0 blocks -> f32 (f16_out = 0) or f16 (f16_out = 1).
 * f32 output is bit-identical to src/dequant.rs:53 `dequantize`; f16 is its RNE
 * rounding. Replaces dequantize_{q4k,q6k,q8_0}_coalesced{,_f16}_kernel
 * (src/kernels_cuda/gemv_q4k.cu:359-448, gemv_q8_0.cu:253-282). */
int rfxq_dequantize(uint32_t ggml_type, const void* blocks, uint64_t num_blocks, void* y, int f16_out,
                    hipStream_t stream);

/* ---- decode GEMV --------------------------------------------------------- */

/* Model::gemv_to (src/model/kernels.rs:1463): y[N] = W . x, x_len == K.
 * Q4_K -> gemv_q4k_r1 path (kernels.rs:2069-2103), Q6_K -> gemv_q6k_r1 path
 * (:2022-2065), Q8_0 -> gemv_q8_0_direct (:1909-1933). */
int rfxq_gemv_to(const float* x, uint64_t x_len, const rfxq_weight* w, float* y, hipStream_t stream);

/* Model::gemv_q4k / gemv_q6k / gemv_q8_0 with `rows` input rows
 * (kernels.rs:2110, :1972, :1874): y[rows][N] = x[rows][K] . W^T with f32
 * activations (the fused few-row GEMV path). */
int rfxq_gemv_rows(const float* x, uint64_t x_len, const rfxq_weight* w, uint32_t rows, float* y,
                   hipStream_t stream);

/* Model::gemv_gather (src/model/kernels.rs:2816-2851): y[j] = (W . x)[row_indices[j]]
 * for j < count, computing only the named rows of W (the System1 candidate
 * LM-head scoring; the reference runs the full-vocab GEMV for a quantized
 * weight and picks rows on the host). row_indices is host memory; y is
 * device memory (count floats); the results equal the full GEMV's at those
 * rows bit for bit. Empty or out-of-range indices fail with the reference's
 * messages. */
int rfxq_gemv_gather(const float* x, uint64_t x_len, const rfxq_weight* w, const uint32_t* row_indices,
                     uint32_t count, float* y, hipStream_t stream);

/* Fused GEMVs of independent weights in one launch (Model::gemv_qkv_to /
 * gemv_gate_up_to, kernels.rs:1761-1823, generalised to any count and mix of
 * Q4_K / Q6_K / Q8_0). */
int rfxq_gemv_batch(const rfxq_gemv_item* items, uint32_t count, hipStream_t stream);

/* A fused GEMV launch whose descriptor table is built and uploaded once and
 * replayed by rfxq_gemv_plan_run (the decode workspace pattern of
 * decode_step_dense_ws, src/model/decode_step.rs:139). */
int rfxq_gemv_plan_create(const rfxq_gemv_item* items, uint32_t count, int device, rfxq_gemv_plan** out);
int rfxq_gemv_plan_run(const rfxq_gemv_plan* plan, hipStream_t stream);
void rfxq_gemv_plan_destroy(rfxq_gemv_plan* plan);

/* ---- prefill GEMM (int8 MMQ) -------------------------------------------- */

/* Q8_1-style activation quantization: xq[rows][k] int8 and xds[rows][k/32]
 * = d_bits | s_bits << 16 (d = amax/127, q = roundf(x/d), s = d*sum(q)). */
int rfxq_quantize_q8_1(const float* x, uint32_t rows, uint32_t k, int8_t* xq, uint32_t* xds, hipStream_t stream);

/* Bytes of workspace rfxq_gemm needs for this weight and row count. */
uint64_t rfxq_gemm_workspace_size(const rfxq_weight* w, uint32_t rows);

/* Model::gemm (src/model/kernels.rs:2197) on a quantized-resident weight:
 * y[rows][N] = x[rows][K] . W^T, on the path rfxq_gemm_policy_for names: one
 * decode GEMV per row (a single row, up to 4 rows, K not a multiple of 256),
 * or activations brought into the f16 layout and the f16-MFMA MMQ kernels
 * for Q4_K, Q6_K and Q8_0 (the int8 Q8_1 layout and kernels with
 * REFLEX_MMQ_F16=0) (replacing gemm_quant_mma,
 * kernels.rs:2262-2340). `workspace` may be NULL (the library then uses its
 * own grow-only per-device buffer: calls on different streams must then not
 * overlap, and a call that would grow it fails under graph capture) or hold
 * rfxq_gemm_workspace_size() bytes. */
int rfxq_gemm(const float* x, uint64_t x_len, const rfxq_weight* w, uint32_t rows, float* y, void* workspace,
              uint64_t workspace_bytes, hipStream_t stream);

/* rfxq_gemm with no device allocation, for callers that cannot allocate
 * (code under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc). It has no counterpart in the reference. Same path, kernels and
 * results as rfxq_gemm with a NULL workspace; the workspace is a fixed
 * 128 MiB device array per GPU (a file-scope __device__ array, held until the
 * process ends), so GEMMs whose workspace (rfxq_gemm_workspace_size) exceeds
 * it fail with RFXQ_ERR_INVALID_INPUT. The device must be initialised first
 * (rfxq_init), which resolves the array's address. Every call on a GPU shares
 * its array and leaves its contents there: calls that overlap on one GPU (on
 * different streams) race. */
int rfxq_gemm_no_alloc(const float* x, uint64_t x_len, const rfxq_weight* w, uint32_t rows, float* y,
                       hipStream_t stream);

/* One GEMM of a grouped launch: y[rows, N] = x[rows, K] . W^T. */
typedef struct rfxq_gemm_item {
    const float* x;
    const rfxq_weight* w;
    float* y;
} rfxq_gemm_item;
typedef struct rfxq_gemm_plan rfxq_gemm_plan;

/* Grouped prefill GEMMs of one row count: the projections that share an
 * input (Model::gemm called for attn_q / attn_k / attn_v on the same normed
 * rows, src/model/dense.rs:1345-1347, and ffn_gate / ffn_up, :1476-1477) as
 * one quantization per distinct x and one MMQ launch per weight type. Same
 * per-item results as rfxq_gemm with REFLEX_QUANT_MMA_SPLITS=1. Uses the
 * library workspace of the current device. */
int rfxq_gemm_batch(const rfxq_gemm_item* items, uint32_t count, uint32_t rows, hipStream_t stream);

/* rfxq_gemm_batch with descriptor tables and activation workspace built once
 * (on `device`) and replayed by rfxq_gemm_plan_run. */
int rfxq_gemm_plan_create(const rfxq_gemm_item* items, uint32_t count, uint32_t rows, int device,
                          rfxq_gemm_plan** out);
int rfxq_gemm_plan_run(const rfxq_gemm_plan* plan, hipStream_t stream);
void rfxq_gemm_plan_destroy(rfxq_gemm_plan* plan);

/* Test hook (the role of q{4,6}k_mma_dequant_check_kernel,
 * src/kernels_cuda/gemm_q_mma.cu:791-838): the MMQ kernel's int32 dot product
 * of every (row, output, 32-block): dots[rows][N][K/32]. For Q6_K the two
 * 16-run int8 scales are folded in: sum_j qa_j * (q6_j - 32) * sc_run(j). */
int rfxq_mmq_block_dots(const int8_t* xq, const uint32_t* xds, uint32_t rows, const rfxq_weight* w, int32_t* dots,
                        hipStream_t stream);

/* ---- fused activation producers (prefill) -------------------------------- */

/* An activation quantized per 32 (Q8_1: int8 values, f16 d and block sum) in
 * every layout the MMQ kernels read, in one caller-owned buffer of
 * rfxq_act_q8_1_size(rows, k) bytes (256-byte aligned; k a multiple of 256).
 * Written by the producers below so that the GEMMs that follow read it
 * directly (no f32 round trip and no separate quantize launch). No reference
 * counterpart: the reference feeds the f32 outputs of its rmsnorm and
 * silu_and_mul into the GEMMs (src/model/dense.rs:1468-1478). */
uint64_t rfxq_act_q8_1_size(uint32_t rows, uint32_t k);

/* Quantize a plain f32 activation [rows][k] into an activation buffer. */
int rfxq_quantize_act_q8_1(const float* x, uint32_t rows, uint32_t k, void* act, hipStream_t stream);

/* Model::rmsnorm (src/kernels_cuda/rmsnorm.cu:18-55, rmsnorm.cuh:17-41) fused
 * with the quantization of its output: y = x / sqrt(mean(x^2) + eps) * weight
 * with the reference's sum order (one thread per row, index order, fused
 * multiply-adds), so the optional f32 output y is bit-identical to the
 * reference kernel's and the buffer equals rfxq_quantize_act_q8_1(y). */
int rfxq_rmsnorm_q8_1(const float* x, const float* weight, uint32_t rows, uint32_t k, float eps, void* act,
                      float* y, hipStream_t stream);

/* Model::silu_and_mul (src/kernels_cuda/silu_and_mul.cu:7-23) fused with the
 * quantization of its output (y optional, equal to rfxq_silu_and_mul's; it
 * must not alias gate or up, which are read once per layout). */
int rfxq_silu_and_mul_q8_1(const float* gate, const float* up, uint32_t rows, uint32_t k, void* act, float* y,
                           hipStream_t stream);

/* An FFN's gate and up GEMMs with Model::silu_and_mul fused into them: from
 * one activation buffer, y = silu(x . Wg^T) * (x . Wu^T) [rows][ffn] (f32,
 * required) and act_out (rfxq_act_q8_1_size(rows, ffn) bytes) =
 * rfxq_quantize_act_q8_1(y), ready for the down GEMM (rfxq_gemm_q8_1).
 * Replaces gemm(gate) + gemm(up) + silu_and_mul (src/model/dense.rs:1476-1478,
 * silu_and_mul.cu:7-23) with the same values: for Q4_K weights on the f16
 * kernels one launch whose tiles hold gate and up columns of the same outputs
 * (no gate / up outputs in memory) and one quantization launch; otherwise
 * the separate GEMMs and rfxq_silu_and_mul_q8_1, with
 * rfxq_gemm_gate_up_silu_workspace_size bytes of workspace (0 for the fused
 * form; NULL uses the library's). No single reference counterpart. gate and
 * up must have one type and shape. */
int rfxq_gemm_gate_up_silu_q8_1(const void* act, uint32_t rows, const rfxq_weight* gate, const rfxq_weight* up,
                                void* act_out, float* y, void* workspace, uint64_t workspace_bytes,
                                hipStream_t stream);
uint64_t rfxq_gemm_gate_up_silu_workspace_size(const rfxq_weight* gate, uint32_t rows);

/* rfxq_gemm / rfxq_gemm_batch from an activation buffer (rows as written).
 * The workspace holds split-K partials only (rfxq_gemm_workspace_size
 * bytes always suffice; NULL uses the library's). */
int rfxq_gemm_q8_1(const void* act, uint32_t rows, const rfxq_weight* w, float* y, void* workspace,
                   uint64_t workspace_bytes, hipStream_t stream);

typedef struct rfxq_gemm_q8_1_item {
    const void* act;
    const rfxq_weight* w;
    float* y;
} rfxq_gemm_q8_1_item;

int rfxq_gemm_q8_1_batch(const rfxq_gemm_q8_1_item* items, uint32_t count, uint32_t rows, hipStream_t stream);

/* rfxq_gemm_plan_create over activation buffers already written (by the
 * producers above): the plan's run launches only the GEMM kernels (and the
 * split-K reduces), no activation pass. Run and destroy it as any plan. The
 * buffers are read at run time, so a producer may rewrite them between runs.
 * No reference counterpart (see rfxq_act_q8_1_size). */
int rfxq_gemm_q8_1_plan_create(const rfxq_gemm_q8_1_item* items, uint32_t count, uint32_t rows, int device,
                               rfxq_gemm_plan** out);

/* ---- MoE ----------------------------------------------------------------- */

/* src/moe.rs:47-98 route_top_k_with_norm on the host: softmax, top-k by
 * probability (ties to the lower index), optional renormalisation. */
int rfxq_route_top_k(const float* logits, uint32_t n, uint32_t k, int normalize, uint32_t* expert, float* weight);

/* Model::quant_expert_weight (kernels.rs:2656-2694): expert e's 2-D slice of a
 * stacked [in, out, E] quantized tensor. */
int rfxq_quant_expert_weight(const rfxq_weight* w, uint32_t expert, rfxq_weight* out);

/* Model::expert_gemv / expert_gemm (src/model/dense.rs:1086-1115). */
int rfxq_expert_gemv(const float* x, uint64_t x_len, const rfxq_weight* w, uint32_t expert, float* y,
                     hipStream_t stream);
int rfxq_expert_gemm(const float* x, uint64_t x_len, const rfxq_weight* w, uint32_t expert, uint32_t rows, float* y,
                     void* workspace, uint64_t workspace_bytes, hipStream_t stream);

/* moe_gather_kernel / moe_scatter_add_kernel (src/kernels_cuda/elementwise.cu:175-222)
 * and silu_and_mul_kernel (src/kernels_cuda/silu_and_mul.cu:7-23). */
int rfxq_moe_gather(const float* src, const uint32_t* perm_row, float* dst, uint32_t num, uint32_t hidden,
                    hipStream_t stream);
int rfxq_moe_scatter_add(const float* src, const uint32_t* dest_row, const float* weight, float* dst, uint32_t num,
                         uint32_t hidden, hipStream_t stream);
int rfxq_silu_and_mul(const float* gate, const float* up, float* out, uint64_t n, hipStream_t stream);

/* Model::moe_ffn_grouped (src/model/dense.rs:1509-1559): route every row on the
 * host (route_top_k_with_norm, weights scaled by weight_scale), then run all
 * experts' gate/up MMQ as one grouped launch, SiLU*up, the down MMQ as one
 * grouped launch and a fixed-order weighted combine into out[rows][hidden]
 * (overwritten). gate/up: [hidden, ffn, E]; down: [ffn, hidden, E]. One
 * host-to-device copy of the routing table; no per-expert launches. Up to 4
 * rows (with 4 <= expert_count <= 1024 and top_k <= 64) run every routed pair
 * as GEMVs planned on the device from the copied routing, the launches of
 * rfxq_moe_ffn_grouped_device. */
int rfxq_moe_ffn_grouped(const float* x, uint32_t rows, uint32_t hidden, const float* router_logits_host,
                         uint32_t expert_count, uint32_t top_k, int normalize, float weight_scale,
                         const rfxq_weight* gate, const rfxq_weight* up, const rfxq_weight* down, float* out,
                         hipStream_t stream);

/* ---- MoE with device-side routing --------------------------------------- */

/* route_top_k_with_norm (src/moe.rs:47-98) for `tokens` rows of device
 * logits [tokens][expert_count]: expert ids and weights (times
 * weight_scale) [tokens][top_k] in selection order, in device memory. The
 * softmax sum is taken in a different order than the host's, so weights can
 * differ from route_top_k's in the last bit. expert_count <= 1024, top_k <= 64. */
int rfxq_moe_route_device(const float* logits, uint32_t tokens, uint32_t expert_count, uint32_t top_k,
                          int normalize, float weight_scale, int32_t* idx, float* weights, hipStream_t stream);

/* rfxq_moe_ffn_grouped with the router logits in device memory: routing,
 * grouping by expert and the GEMV or MMQ descriptor tables are built on the
 * device (the reference copies the logits to the host and uploads
 * per-expert row lists, src/model/dense.rs:1539-1546, 1602-1605), so the
 * call adds no host synchronisation and no host-to-device copy. Up to 4
 * tokens run every routed pair as GEMVs, as the host-routed path does; more
 * take the grouped MMQ path (row tiles per GEMM by the expert groups' average
 * rows and the waves of workgroups their tiles need). Requires
 * 4 <= expert_count <= 1024, top_k <= 64 and rows * top_k <= 16384.
 * Routing errors of the host path (non-finite softmax sums) are not
 * reported: such tokens get non-finite outputs. */
int rfxq_moe_ffn_grouped_device(const float* x, uint32_t rows, uint32_t hidden, const float* router_logits,
                                uint32_t expert_count, uint32_t top_k, int normalize, float weight_scale,
                                const rfxq_weight* gate, const rfxq_weight* up, const rfxq_weight* down, float* out,
                                hipStream_t stream);

/* ---- GGUF files (the on-disk path) ---------------------------------------- */

/* GgufFile (src/gguf.rs:183-334): the file memory-mapped and parsed (magic,
 * version, metadata with nested arrays, tensor infos, data section at the
 * `general.alignment` boundary, default 32). Errors: RFXQ_ERR_IO (open /
 * map), RFXQ_ERR_GGUF (format, with the reference's messages). Tensor data
 * pointers point into the mapping and live until rfxq_gguf_close. */
typedef struct rfxq_gguf rfxq_gguf;
int rfxq_gguf_open(const char* path, rfxq_gguf** out);
void rfxq_gguf_close(rfxq_gguf* file);
uint32_t rfxq_gguf_version(const rfxq_gguf* file);
uint64_t rfxq_gguf_tensor_count(const rfxq_gguf* file);
/* tensor_info (gguf.rs:281): the first tensor of that name */
int rfxq_gguf_find_tensor(const rfxq_gguf* file, const char* name, uint64_t* index);
/* dims: 4 entries, unused ones 1 */
int rfxq_gguf_tensor_info(const rfxq_gguf* file, uint64_t index, const char** name, uint32_t* n_dims,
                          uint64_t* dims, uint32_t* ggml_type, uint64_t* offset);
/* tensor_bytes (gguf.rs:310-334): the tensor's bytes in the mapping */
int rfxq_gguf_tensor_data(const rfxq_gguf* file, uint64_t index, const void** data, uint64_t* bytes);
int rfxq_gguf_meta_u64(const rfxq_gguf* file, const char* key, uint64_t* out);
int rfxq_gguf_meta_f64(const rfxq_gguf* file, const char* key, double* out);
int rfxq_gguf_meta_str(const rfxq_gguf* file, const char* key, const char** out);
int rfxq_gguf_meta_array_len(const rfxq_gguf* file, const char* key, uint64_t* out);
/* QuantArena (src/model/loading.rs:266-317): bytes of one device allocation
 * holding the listed tensors at 256-byte aligned offsets (0 on a bad index
 * or range), and the upload into it; weights[j] describes tensor j as the
 * kernels take it (GGUF shape [in, out(, experts)], raw blocks). */
uint64_t rfxq_gguf_arena_size(const rfxq_gguf* file, const uint64_t* indices, uint32_t count);
int rfxq_gguf_upload(const rfxq_gguf* file, const uint64_t* indices, uint32_t count, void* arena,
                     uint64_t arena_bytes, rfxq_weight* weights, hipStream_t stream);

#ifdef __cplusplus
}
#endif
#endif /* RFXQ_H */
