/*
 * libllmoe -- LLaDA2 routed-expert MoE layer on MI355X (gfx950), C ABI.
 *
 * One layer object holds one MoE layer's expert weights (routed experts 0..E-1 plus an optional shared expert
 * at index E) resident in HBM, its router, and a workspace sized for `max_tokens` tokens. Every compute call
 * takes DEVICE pointers, is asynchronous on the given HIP stream (NULL = the default stream), performs no host
 * synchronisation, no allocation and no memset, and is therefore capturable in a HIP graph. Work-item counts
 * are produced and consumed on the device.
 *
 * Errors: every call returns LLMOE_OK (0) or a negative LLMOE_E* code; llmoe_last_error() returns the message
 * of the calling thread's last failure. Nothing exits the process.
 *
 * Threading: a layer object is not thread-safe (its workspace is shared by its calls); serialise calls per
 * layer, as the reference serialises llada_generate with a mutex (engine/libllada.cu:30). Distinct layer
 * objects may be used concurrently on distinct streams.
 *
 * Reference interfaces replaced (patrickbdevaney/llada2-orin-cuda; the reference exposes the MoE path as
 * in-process C++ below its whole-model C ABI engine/libllada.cu:13-52):
 *   llmoe_layer_create    Engine::load's expert part: ExpertTable + relayout_matrix (engine/engine.cu:206-224,
 *                         engine/moe_i8.cu:48-53, :93-121)
 *   llmoe_layer_load      the same from the on-disk model directory (read_index + Engine::load,
 *                         engine/engine.cu:54-75, :166-224)
 *   llmoe_quantize_a8     ops::quant_rows_q8 / quant_row_smem (engine/ops.cu:40-66, :127-135)
 *   llmoe_route           ops::router_mma + ops::route_schedule / route_batch_select/plan/place
 *                         (engine/ops.cu:137-205, :223-423)
 *   llmoe_dispatch        the host counting sort of engine/tests/test_moe_i8.cu:73-98 (externally routed)
 *   llmoe_experts         gemm<..,0> -> fwht512_q8 -> gemm<..,1> -> combine (engine/engine.cu:461-478,
 *                         engine/moe_i8.cu:408-515)
 *   llmoe_experts_norm    llmoe_experts + ops::moe_combine_norm (engine/ops.cu:507-549): un-rotation, residual,
 *                         next-layer RMSNorm / rotation / A8
 *   llmoe_layer_forward   the MoE half of Engine::layer_step / Engine::prefill (engine/engine.cu:445-479,
 *                         :616-649), without the norm/rotation before it and the un-rotation after it
 *   llmoe_layer_forward_norm  the same with ops::moe_combine_norm's epilogue (engine/ops.cu:507-549): the MoE half
 *                         of Engine::layer_step up to the next layer's A8 input
 */
#ifndef LLMOE_H
#define LLMOE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define LLMOE_OK 0
#define LLMOE_EINVAL (-1)   /* bad argument or shape */
#define LLMOE_ENOMEM (-2)   /* device or host allocation failed */
#define LLMOE_EHIP (-3)     /* a HIP runtime call failed */
#define LLMOE_ESTATE (-4)   /* call order: llmoe_experts before llmoe_route / llmoe_dispatch for this T */

typedef struct llmoe_layer llmoe_layer;
typedef void* llmoe_stream; /* hipStream_t */

typedef struct {
    int hidden;          /* H, must be 2048 (LLaDA2.2-mini; the GEMM geometry is compiled for it) */
    int inter;           /* I, must be 512 (FWHT-512 on the down input) */
    int n_experts;       /* E routed experts, <= 256 */
    int top_k;           /* K experts per token, <= 8 */
    int pool;            /* C: per-block expert pool (48 shipped, engine/ops.cu:257); >= E disables it */
    int block;           /* tokens per routing block (32, the diffusion block); <= 32 */
    float routed_scale;  /* w = score / sum(score) * routed_scale (2.5, engine/engine.cu:142) */
    int has_shared;      /* expert index E is a shared expert, applied to every token with weight 1 */
    int max_tokens;      /* workspace capacity in tokens */
} llmoe_layer_desc;

/* Create a layer from packlib format-"i8" expert matrices (quant/packlib.py:140-197) in HOST memory.
 *   blob            packed matrices; gate_up of expert e at gu_off[e] ([2I, H], rows permuted by gu_row_perm,
 *                   quant/packlib.py:98-102), down at d_off[e] ([H, I])
 *   gu_off, d_off   [E + has_shared] byte offsets into blob
 *   bits            [E + has_shared] 2, 3, 4 or 8
 *   router_w        [H, E] fp32 router matrix (k-major), or NULL (then only logits routing is available)
 *   router_bias     [E] fp32 expert bias (required)
 * The library copies the weights to HBM and rewrites them in place into its MFMA operand layout. */
int llmoe_layer_create(const llmoe_layer_desc* desc, const void* blob, size_t blob_bytes, const uint64_t* gu_off,
                       const uint64_t* d_off, const int8_t* bits, const float* router_w, const float* router_bias,
                       llmoe_layer** out);
int llmoe_layer_destroy(llmoe_layer* layer);

/* A8: x fp32 [rows, cols] -> q int8 [rows, cols] (logical column order), s fp32 [rows, cols/128],
 * sum int32 [rows, cols/128]; symmetric per (row, 128-group), s = max(max|x| / 127, 1e-30),
 * q = clamp(rint(x / s), +-127). cols % 512 == 0. */
int llmoe_quantize_a8(const float* x, int rows, int cols, int8_t* q, float* s, int32_t* sum, llmoe_stream stream);

/* Routing + dispatch for T tokens. Exactly one of x (fp32 [T, H], router input: logits = x Wr) and logits
 * (fp32 [T, E]) is non-NULL. Results stay in the layer workspace (llmoe_layer_buffers). */
int llmoe_route(llmoe_layer* layer, const float* x, const float* logits, int T, llmoe_stream stream);

/* Dispatch for externally routed tokens: topk int32 [T, K] (K DISTINCT experts per token), topw fp32 [T, K]. */
int llmoe_dispatch(llmoe_layer* layer, const int32_t* topk, const float* topw, int T, llmoe_stream stream);

/* Expert stage for the routing last set for the same T: gate_up -> FWHT-512 + A8 -> down -> combine.
 * xq/xs/xsum: A8 activations of the T tokens (llmoe_quantize_a8 layout). out: fp32 [T, H]
 *   out[t] = sum_k w[t,k] expert_k(x_t) (+ shared(x_t)), summed in rank order, shared last. */
int llmoe_experts(llmoe_layer* layer, const int8_t* xq, const float* xs, const int32_t* xsum, int T, float* out,
                  llmoe_stream stream);

/* llmoe_experts with the combine's consumer fused in (engine/ops.cu:507-549, moe_combine_norm): the combined
 * expert output, still in the rotated basis, is un-rotated and added to the residual stream, and the next layer's
 * input norm is applied:
 *   h[t] += (FWHT2048(sum_k Y_k) * signs) / sqrt(2048)                     (Q^T = H diag(signs) / sqrt(2048))
 *   (q_next, s_next, sum_next) = A8(FWHT2048((h[t] / rms(h[t], eps)) * signs) / sqrt(2048))
 * signs fp32 [2048] of +-1 (the residual rotation), h fp32 [T, 2048] in/out, q_next int8 [T, 2048], s_next fp32
 * [T, 16], sum_next int32 [T, 16] (the llmoe_quantize_a8 layout; RMSNorm gamma is folded into the next
 * layer's weights). hidden must be 2048. */
int llmoe_experts_norm(llmoe_layer* layer, const int8_t* xq, const float* xs, const int32_t* xsum, int T,
                       const float* signs, float eps, float* h, int8_t* q_next, float* s_next, int32_t* sum_next,
                       llmoe_stream stream);

/* llmoe_experts without any device memory of the layer's own for the expert stage's intermediates (Z, its A8,
 * the slot outputs Y): they live in one static device array per GPU, LLMOE_SCRATCH_BYTES bytes, held by each GPU
 * the library runs on until the process ends. No counterpart in the reference: for callers that cannot allocate
 * (code under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc) and for stacks of layers
 * that share one set of intermediates. The call allocates nothing and performs no memset; nothing in the array
 * needs to start at zero (every element a call reads was written earlier in that call). T <= LLMOE_SCRATCH_MAX_TOKENS
 * (larger T: LLMOE_EINVAL); hidden 2048, inter 512, top_k <= 8. Every call on one GPU shares the array: calls that
 * overlap on one GPU (other streams, other threads) race and must be serialised by the caller. Same results as
 * llmoe_experts. */
#define LLMOE_SCRATCH_MAX_TOKENS 64
#define LLMOE_SCRATCH_BYTES 5621760u
int llmoe_experts_scratch(llmoe_layer* layer, const int8_t* xq, const float* xs, const int32_t* xsum, int T,
                          float* out, llmoe_stream stream);

/* Whole layer: A8(x) -> route (x Wr, or the given logits) -> experts -> out. x fp32 [T, H]. At decode (T <= block)
 * the slot plan is built inside the gate_up GEMM rather than by a dispatch kernel; the results and the buffers
 * (llmoe_layer_buffers) are the same as route + experts. */
int llmoe_layer_forward(llmoe_layer* layer, const float* x, const float* logits, int T, float* out,
                        llmoe_stream stream);

/* llmoe_layer_forward with the epilogue of llmoe_experts_norm instead of writing out: route from x (or the given
 * logits), the experts, then the combine, un-rotation, residual add into h, and the next layer's RMSNorm / rotation
 * / A8 into q_next, s_next, sum_next (layouts as llmoe_experts_norm; hidden must be 2048). At decode the slot plan
 * is built inside the gate_up GEMM, as in llmoe_layer_forward; same results as llmoe_route + llmoe_experts_norm. */
int llmoe_layer_forward_norm(llmoe_layer* layer, const float* x, const float* logits, int T, const float* signs,
                             float eps, float* h, int8_t* q_next, float* s_next, int32_t* sum_next,
                             llmoe_stream stream);

/* Numerics of a layer's expert stage (default LLMOE_NUMERICS_EXACT).
 *   EXACT: every stage follows one fixed fp32 operation sequence, so results are bit-identical run to run and to
 *          the CPU restatement of the reference. The routing sigmoid uses a degree-7 polynomial exp and a correctly
 *          rounded divide; the gate_up SiLU a degree-5 polynomial exp with exact ldexp scaling and a reciprocal by
 *          three Newton steps; fp32 -> fp16 is integer round-to-nearest-even.
 *   FAST:  the SiLU of gate_up uses the hardware exp, reciprocal and fp16 conversion -- the precision of the
 *          reference's own __expf / __fdividef / __float2half (engine/moe_i8.cu:221) -- and, with several routing
 *          blocks (T > block), the down GEMM stores each slot output w acc rounded to fp16 (nearest even) for the
 *          combine, which halves the slot outputs' HBM round trip (|w acc| must stay below 65504). Z then differs from EXACT by at most one fp16 rounding
 *          step; the int32 expert products and every later stage are computed exactly as in EXACT from that Z (up to
 *          the slot outputs' fp16 rounding), and the layer output agrees with EXACT within the contract's 1e-3
 *          tolerance.
 * Takes effect from the next llmoe_experts / llmoe_experts_norm / llmoe_layer_forward call on the layer. */
#define LLMOE_NUMERICS_EXACT 0
#define LLMOE_NUMERICS_FAST 1
int llmoe_layer_set_numerics(llmoe_layer* layer, int mode);

/* Device pointers of the layer workspace (valid until destroy), for inspection and tests. Slot s in
 * [0, T K) is a routed (token, expert) pair, expert-major then token-ascending; slot T K + t is token t's
 * shared-expert slot. */
typedef struct {
    int8_t* xq; float* xs; int32_t* xsum;              /* A8 of the layer input        [T, H], [T, H/128] */
    float* logits_part;                                /* router partials              [8, T, E] */
    int32_t* topk; float* topw;                        /*                              [T, K] */
    int32_t* count; int32_t* start;                    /* slots per routed expert      [E] */
    int32_t* slot_token; float* slot_weight;           /*                              [S] */
    int32_t* tok_slots;                                /* [T, K + 1] (last: shared slot, -1 if none) */
    int32_t* items; int32_t* n_items;                  /* gate_up work units {expert, slot0, ntok, row block};
                                                          n_items[0] / [1]: gate_up / down unit counts */
    uint16_t* Z;                                       /* fp16 SiLU(g) u               [S, I] */
    int8_t* zq; float* zs; int32_t* zsum;              /* A8(Z H512)                   [S, I], [S, I/128] */
    float* Y;                                          /* weighted expert outputs      [S, H]
                                                          (fp16 bits [S, H] after a LLMOE_NUMERICS_FAST call
                                                          with T > block) */
    int ntok;                                          /* tokens per work item of the last dispatch */
    int max_items;                                     /* work-item capacity of the last dispatch */
} llmoe_buffers;
int llmoe_layer_buffers(const llmoe_layer* layer, llmoe_buffers* out);

/* Expert weight bytes resident in HBM (the weight-stream bytes of a full pass over every expert). */
int llmoe_layer_weight_bytes(const llmoe_layer* layer, size_t* bytes);

/* Exact int32 group products of one expert matrix (test entry; the same MFMA core as llmoe_experts):
 *   P[n, r, g] = sum_{k in group g} code[r, k] xq[n, k] - zero[r, g] xsum[n, g]
 * which: 0 = gate_up ([2I, H], r in packlib row order), 1 = down ([H, I]). xq int8 [n, Kw], xsum [n, Kw/128],
 * n <= 64. P int32 [n, R, Kw/128]. */
int llmoe_group_products(llmoe_layer* layer, int expert, int which, const int8_t* xq, const int32_t* xsum, int n,
                         int32_t* P, llmoe_stream stream);

/* Self-test of the device's fp32 -> fp16 conversion (test entry; no counterpart in the reference): every finite fp32
 * bit pattern through the hardware conversion the kernels use (v_cvt_f16_f32) and through round-to-nearest-even
 * spelled out in integer ops (the definition the CPU checker restates); *mismatches = the number of inputs on which
 * they differ (0 on gfx950). Synchronous; takes a fraction of a second. */
int llmoe_selftest_f16(uint64_t* mismatches);

/* Per-stage timing (the analogue of Engine::mark / prof_collect, engine/engine.cu:385-407, enabled there by
 * PROF=1): while enabled, every stage of the layer's calls is bracketed by HIP events on the call's stream.
 * Not for use under graph capture. llmoe_layer_stage_ms waits for the last recorded stage and returns, per
 * stage, the milliseconds of its latest run (-1 if it has not run since profiling was enabled).
 * Stages: LLMOE_STAGE_* below. */
#define LLMOE_STAGE_QUANT 0
#define LLMOE_STAGE_ROUTER 1
#define LLMOE_STAGE_ROUTE 2
#define LLMOE_STAGE_DISPATCH 3
#define LLMOE_STAGE_GATE_UP 4
#define LLMOE_STAGE_FWHT 5
#define LLMOE_STAGE_DOWN 6
#define LLMOE_STAGE_COMBINE 7
#define LLMOE_N_STAGES 8
int llmoe_layer_set_profiling(llmoe_layer* layer, int enabled);
int llmoe_layer_stage_ms(llmoe_layer* layer, float* ms);

/* Re-launch one expert stage of the latest llmoe_experts / llmoe_experts_norm call (LLMOE_STAGE_GATE_UP, _FWHT,
 * _DOWN or _COMBINE) `reps` times back to back between two HIP events on `stream`, and return the average
 * milliseconds per launch (the kernel's steady-state duration). The stages are idempotent except the combine of
 * an llmoe_experts_norm call, which adds into h again on every repeat. Waits for completion. When the latest call
 * had one routing block (T <= block), FWHT-512 + A8 ran inside the down GEMM: LLMOE_STAGE_FWHT then returns
 * LLMOE_ESTATE and its cost is part of LLMOE_STAGE_DOWN. */
int llmoe_layer_time_stage(llmoe_layer* layer, int stage, int reps, llmoe_stream stream, float* avg_ms);

/* As llmoe_layer_time_stage over n layers launched in turn (layer 0, 1, .., n-1, repeated `reps` times): with
 * more weight bytes than the GPU's last-level cache (256 MB on MI355X) every launch streams from HBM.
 * avg_ms = milliseconds per launch. */
int llmoe_layers_time_stage(llmoe_layer* const* layers, int n, int stage, int reps, llmoe_stream stream,
                            float* avg_ms);

/* Load the MoE half of layer `layer` from the reference's model directory (engine/engine.cu:54-75, :166-224):
 * engine.idx (C config, T tensors, E experts, F file sizes, quant/s07c_index.py), the routed experts of
 * experts_L<layer>.bin, the shared expert ("gate_up", "down" of nonexpert_L<layer>.bin, packlib i8 at C
 * nonexpert_bits), the router (small.bin "L<layer>.router", bf16 [E, H]) and the expert bias (small.bin
 * "L<layer>.expert_bias", fp32 [E]); pool = C expert_capacity (48), block = C block_size (32). Pruned experts
 * (bits 0) are rejected. Then as llmoe_layer_create with max_tokens. */
int llmoe_layer_load(const char* model_dir, int layer, int max_tokens, llmoe_layer** out);

/* The residual-rotation signs (small.bin "signs", fp32 [n], Q = diag(signs) H / sqrt(n)) into host memory. */
int llmoe_model_signs(const char* model_dir, float* signs, int n);

/* Dense W.A8 projection (engine/engine.cu:380-383, :425, :434: qkv, the attention output and the lm_head run
 * through the expert GEMM as one "expert" holding every token; KAT engine/tests/gen_dense_case.py). One [rows, k]
 * matrix of b-bit codes in packlib "i8" (quant/packlib.py), rows in packlib order; k = 2048, rows a multiple of
 * 256, bits 2 / 3 / 4 / 8. The blob is read once, relaid out on the device and not kept. */
typedef struct llmoe_dense llmoe_dense;
int llmoe_dense_create(int rows, int k, int bits, const uint8_t* blob, size_t blob_bytes, int max_tokens,
                       llmoe_dense** out);
int llmoe_dense_destroy(llmoe_dense* dense);

/* y[t, r] = sum over the 16 groups g (ascending) of the fma chain of scale_w[r, g] * xs[t, g] and the exact int32
 * group product (the expert GEMMs' epilogue), for the T <= max_tokens A8 rows (xq int8 [T, 2048], xs fp32 [T, 16],
 * xsum int32 [T, 16], the llmoe_quantize_a8 layout); accumulate != 0: y += that (the residual add of
 * engine/engine.cu:434). y fp32 [T, rows] on the device; asynchronous on `stream`. */
int llmoe_dense_forward(llmoe_dense* dense, const int8_t* xq, const float* xs, const int32_t* xsum, int T, float* y,
                        int accumulate, llmoe_stream stream);

/* Message of the calling thread's last error ("" if none). */
const char* llmoe_last_error(void);

#ifdef __cplusplus
}
#endif
#endif
