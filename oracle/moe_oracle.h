/*
 * CPU oracle for the routed-expert MoE layer -- TEST INFRASTRUCTURE ONLY.
 *
 * This library is the checker the HIP product path is compared against. Only tests/, the smoke() entry of
 * __graft_entry__.py and bench.py's cpu_baseline leg may load it; the product (libllmoe.so) never links or
 * calls it. Every function restates the reference algorithm it cites (paths relative to the reference repo
 * patrickbdevaney/llada2-orin-cuda) in plain C, with one deliberate difference that is shared with the GPU
 * product: transcendental functions are this file's own (orc_exp for the routing sigmoid, orc_silu for the
 * gate_up epilogue), so the GPU can reproduce every fp32 operation bit for bit.
 *
 * Floating-point contract shared with the GPU kernels (compile with -ffp-contract=off):
 *   - every add / mul / div is an IEEE fp32 op, fused multiply-adds only where written as fmaf();
 *   - float -> int rounding is rint() (round half to even);
 *   - fp32 -> fp16 is round to nearest even (orc_f32_to_f16).
 *
 * Pinning status of each function (what checks it independently of this file) is listed in the tests
 * (tests/test_oracle_*.py).
 */
#ifndef LLMOE_ORACLE_H
#define LLMOE_ORACLE_H
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- numeric primitives --------------------------------------------------------------------------------- */
float orc_exp(float x);
float orc_sigmoid(float x);
float orc_silu(float x);
uint16_t orc_f32_to_f16(float x);
float orc_f16_to_f32(uint16_t h);

/* ---- packlib format "i8" (quant/packlib.py:140-234) ---------------------------------------------------- */
int orc_tile_wbytes(int bits);
size_t orc_matrix_bytes(int R, int K, int bits);
void orc_pack_i8(const uint8_t* codes, const uint16_t* scale, const uint8_t* zero, int R, int K, int bits,
                 uint8_t* out);
void orc_unpack_i8(const uint8_t* blob, int R, int K, int bits, uint8_t* codes, uint16_t* scale, uint8_t* zero);
void orc_gu_row_perm(int I, int32_t* perm);

/* ---- A8 activation quantiser (engine/ops.cu:40-66, engine/tests/test_moe_i8.cu:52-71) ------------------- */
void orc_quant_a8(const float* x, int rows, int K, int8_t* q, float* s, int32_t* sum);

/* ---- router (a1, a2) and dispatch (a3) ------------------------------------------------------------------ */
void orc_router_logits(const float* x, const float* Wr, int T, int H, int E, float* logits);
void orc_route(const float* logits, const float* bias, int T, int E, int K, int C, int block, float rscale,
               int32_t* topk, float* topw);
int orc_dispatch(const int32_t* topk, const float* topw, int T, int E, int K, int has_shared, int32_t* count,
                 int32_t* start, int32_t* slot_token, float* slot_weight, int32_t* tok_slots);

/* ---- expert products ------------------------------------------------------------------------------------ */
void orc_group_products(const uint8_t* codes, const uint8_t* zero, int R, int K, const int8_t* xq,
                        const int32_t* xsum, int32_t* P);
void orc_fwht_a8(const uint16_t* Z, int nslots, int8_t* q, float* s, int32_t* sum);
void orc_fwht512_f32(float* v);

typedef struct {
    int H, I, E, K;              /* hidden, intermediate, routed experts, top-k */
    int has_shared;              /* expert index E is the shared expert */
    const uint8_t* blob;         /* packlib-i8 matrices */
    const uint64_t* gu_off;      /* [E + 1] byte offset of gate_up (rows permuted by gu_row_perm) */
    const uint64_t* d_off;       /* [E + 1] byte offset of down */
    const int8_t* bits;          /* [E + 1] 2 / 3 / 4 / 8 */
} orc_layer;

/* Expert stage for all slots (routed slots [0, T*K), shared slots [T*K, T*K + T)): gate_up -> Z (fp16 bits),
 * FWHT-512 + A8 -> (zq, zs, zsum), down -> Y, combine -> out. Any output pointer may be NULL except out.
 * nthreads: OpenMP threads over experts (<= 0: library default). Returns 0 or a negative error code. */
int orc_experts(const orc_layer* L, const int8_t* xq, const float* xs, const int32_t* xsum, int T,
                const int32_t* count, const int32_t* start, const int32_t* slot_token, const float* slot_weight,
                const int32_t* tok_slots, uint16_t* Z, int8_t* zq, float* zs, int32_t* zsum, float* Y, float* out,
                int nthreads);

/* orc_experts from the gate_up outputs Z [S, I] (fp16 bits) of every slot: FWHT-512 + A8, down, combine. yhalf != 0:
 * each slot output is rounded to fp16 (nearest even) before the combine -- the build's fast-numerics Y -- and Y
 * returns those values as fp32. */
int orc_experts_from_z(const orc_layer* L, const uint16_t* Z, int yhalf, int T, const int32_t* count,
                       const int32_t* start, const int32_t* slot_token, const float* slot_weight,
                       const int32_t* tok_slots, int8_t* zq, float* zs, int32_t* zsum, float* Y, float* out,
                       int nthreads);

/* Independent fp64 dequantize-then-matmul reference (engine/tests/gen_moe_case.py:77-93): acc[t] =
 * sum_k w_k * d(a8(fp16(SiLU(g x') * (u x')) H512)) with x' = a8(x) dequantised, plus the shared expert
 * with weight 1. topk / topw give the routing. */
int orc_reference_f64(const orc_layer* L, const float* x, int T, const int32_t* topk, const float* topw,
                      double* out, int nthreads);

/* Combine + un-rotation + residual add + the next layer's RMSNorm, rotation and A8 (engine/ops.cu:507-549), H = 2048:
 * h [T, 2048] is updated in place; q/s/sum receive the next layer's A8 input. */
/* Dense W.A8 projection (engine/engine.cu:380-383, :425, :434; the expert GEMM's integer core and fp32 epilogue
 * with one matrix): y[t, r] = row_epilogue(P[r, :, t]) for the [R, K] packlib-i8 matrix, or y += that. */
int orc_dense(const uint8_t* blob, int R, int K, int bits, const int8_t* xq, const float* xs, const int32_t* xsum,
              int T, float* y, int accumulate, int nthreads);

void orc_combine_norm(const float* Y, const int32_t* tok_slots, int T, int nk, int K1, const float* signs, float eps,
                      float* h, int8_t* q, float* s, int32_t* sum);

#ifdef __cplusplus
}
#endif
#endif
