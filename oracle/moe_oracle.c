/*
 * CPU oracle for the routed-expert MoE layer -- TEST INFRASTRUCTURE ONLY (see moe_oracle.h).
 *
 * Restates, in plain C, the reference's algorithm for this path. Citations are to the reference repository
 * patrickbdevaney/llada2-orin-cuda:
 *   format "i8"            quant/packlib.py:140-234 (pack_matrix_i8 / unpack_matrix_i8), :98-102 (gu_row_perm)
 *   A8 quantiser           engine/ops.cu:40-66 (quant_row_smem), engine/tests/gen_moe_case.py:24-29 (a8)
 *   router logits          engine/ops.cu:137-205 (router_mma: K split in 8 partials, fixed-order sum)
 *   routing                engine/ops.cu:256-327 (route_core), quant/s03_teacher_pass.py:132-146 (route)
 *   dispatch               engine/ops.cu:333-370 (route_schedule), :384-423 (route_batch_plan/place)
 *   expert integer core    engine/moe_i8.cu:1-14 (P_g = sum q xq - z Sxq), :364-383 (fp32 epilogue per group)
 *   SiLU -> fp16           engine/moe_i8.cu:219-221
 *   FWHT-512 + A8          engine/moe_i8.cu:444-502
 *   down + routing weight  engine/moe_i8.cu:222-231
 *   combine                engine/moe_i8.cu:504-515
 *   fp64 reference         engine/tests/gen_moe_case.py:20-36, 77-93; quant/quantlib.py:138-142
 *
 * Build with -ffp-contract=off: the fp32 operation sequence here is the contract the GPU kernels reproduce.
 */
#include "moe_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

#define GROUP 128
#define META 48

/* ------------------------------------------------------------------------------------------------------------
 * numeric primitives
 * ------------------------------------------------------------------------------------------------------------ */

static inline float bits_f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }
static inline uint32_t f_bits(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }

/* 2^k for k in [-126, 127], built from its exponent field. */
static inline float pow2i(int k) { return bits_f((uint32_t)(k + 127) << 23); }

/* exp(x): Cody-Waite reduction x = n ln2 + r (ln2 split hi + lo, hi with 12 trailing zero bits so n * hi is
 * exact for |n| <= 2^11), Taylor polynomial of degree 7 on |r| <= ln2 / 2 (truncation error < 2^-27 relative),
 * scaling by 2^n in two exact power-of-two factors. The reference uses CUDA's __expf (engine/ops.cu:271,
 * engine/moe_i8.cu:221); this build defines its own so CPU and GPU agree bit for bit. */
float orc_exp(float x) {
    if (x != x) return x;
    if (x > 88.72283935546875f) return INFINITY;
    if (x < -103.97208404541016f) return 0.0f;
    const float n = rintf(x * 1.44269502162933349609375f);
    float r = fmaf(n, -0.693145751953125f, x);
    r = fmaf(n, -1.428606765330187045037746429443359375e-06f, r);
    float p = 1.98412701138295233249664306640625e-04f;      /* 1/7! */
    p = fmaf(p, r, 1.38888892345130443572998046875e-03f);     /* 1/6! */
    p = fmaf(p, r, 8.33333376795053482055664062500e-03f);     /* 1/5! */
    p = fmaf(p, r, 4.16666679084300994873046875000e-02f);     /* 1/4! */
    p = fmaf(p, r, 1.66666671633720397949218750000e-01f);     /* 1/3! */
    p = fmaf(p, r, 0.5f);
    p = fmaf(p, r, 1.0f);
    p = fmaf(p, r, 1.0f);
    const int ni = (int)n, e1 = ni / 2, e2 = ni - e1;
    return (p * pow2i(e1)) * pow2i(e2);
}

float orc_sigmoid(float x) { return 1.0f / (1.0f + orc_exp(-x)); }
/* SiLU of the gate_up epilogue (its result is multiplied by u and rounded to fp16): exp(-g) by Cody-Waite with one
 * ln2 constant and a degree-5 Taylor polynomial, exact scaling by ldexp, 1 / (1 + e) by three Newton steps from a
 * bit-pattern seed; the exp argument clamped to [-104, 80], which keeps every step finite. */
float orc_silu(float g) {
    const float x = fminf(fmaxf(-g, -104.0f), 80.0f);
    const float n = rintf(x * 1.44269502162933349609375f);
    const float r = fmaf(n, -0.693147182464599609375f, x);
    float p = 8.33333376795053482055664062500e-03f;           /* 1/5! */
    p = fmaf(p, r, 4.16666679084300994873046875000e-02f);      /* 1/4! */
    p = fmaf(p, r, 1.66666671633720397949218750000e-01f);      /* 1/3! */
    p = fmaf(p, r, 0.5f);
    p = fmaf(p, r, 1.0f);
    p = fmaf(p, r, 1.0f);
    const float d = 1.0f + ldexpf(p, (int)n);
    float q = bits_f(0x7EF311C3u - f_bits(d));
    for (int i = 0; i < 3; ++i) q = fmaf(q, fmaf(-d, q, 1.0f), q);
    return g * q;
}

/* fp32 -> fp16, round to nearest even, overflow to inf, subnormals kept. */
uint16_t orc_f32_to_f16(float f) {
    const uint32_t x = f_bits(f);
    const uint16_t sign = (uint16_t)((x >> 16) & 0x8000u);
    const uint32_t ax = x & 0x7fffffffu;
    if (ax >= 0x7f800000u) return (uint16_t)(sign | 0x7c00u | (ax > 0x7f800000u ? 0x200u : 0u));
    if (ax >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u);          /* >= 65520 rounds to inf */
    if (ax < 0x38800000u) {                                              /* below 2^-14: subnormal half */
        const uint32_t m = (uint32_t)rintf(bits_f(ax) * 16777216.0f);  /* exact scale by 2^24 */
        return (uint16_t)(sign | m);
    }
    const uint32_t mant = ax & 0x7fffffu;
    uint32_t h = ((uint32_t)((int)(ax >> 23) - 127 + 15) << 10) | (mant >> 13);
    const uint32_t rem = mant & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) ++h;
    return (uint16_t)(sign | h);
}

float orc_f16_to_f32(uint16_t h) {
    const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    const uint32_t e = (h >> 10) & 0x1f, m = h & 0x3ffu;
    if (e == 0) {
        const float v = (float)m * 5.9604644775390625e-08f;           /* m * 2^-24, exact */
        return (h & 0x8000u) ? -v : v;
    }
    if (e == 31) return bits_f(sign | 0x7f800000u | (m << 13));
    return bits_f(sign | ((e - 15 + 127) << 23) | (m << 13));
}

/* ------------------------------------------------------------------------------------------------------------
 * packlib format "i8" (quant/packlib.py:140-234)
 *
 * A matrix [R, K] is cut into strips of 16 rows, a strip into K/128 tiles (16 rows x one 128-column group).
 * Inside a tile, lane l (g = l/4, t = l%4) holds for k32-step j the registers r = 0..3:
 *   r = 0: row g,   cols 32j + 4t + b        r = 1: row g + 8, same cols
 *   r = 2: row g,   cols 32j + 16 + 4t + b   r = 3: row g + 8, same cols          (b = byte 0..3)
 * Plane storage (bytes inside the tile's code area):
 *   8-bit: word (j, r) of lane l at ((j*32 + l)*4 + r)*4, byte b = code
 *   4-bit: word 2j + (r/2) -> uint4 u = w/4, word-in-uint4 w%4 at ((u*32 + l)*4 + w%4)*4; byte b low nibble =
 *          register 2(r/2), high nibble = register 2(r/2) + 1
 *   2-bit: word j at (l*4 + j)*4; bits 8b + 2r .. 8b + 2r + 1 = low two bits of code (j, r, b)
 *   3-bit: the 2-bit plane plus a high plane at 512 + (l*2 + j/2)*4; bit 8b + 4(j%2) + r = bit 2 of the code
 * followed by 16 fp16 scales (rows 0..15) and 16 u8 zeros. Dequantised weight = (code - zero) * scale.
 * ------------------------------------------------------------------------------------------------------------ */

int orc_tile_wbytes(int bits) { return bits == 8 ? 2048 : bits == 4 ? 1024 : bits == 3 ? 768 : bits == 2 ? 512 : -1; }

size_t orc_matrix_bytes(int R, int K, int bits) {
    return (size_t)(R / 16) * (size_t)(K / GROUP) * (size_t)(orc_tile_wbytes(bits) + META);
}

/* row / column of (lane, j, r, b) inside a tile */
static inline int tile_row(int lane, int r) { return (lane >> 2) + 8 * (r & 1); }
static inline int tile_col(int lane, int j, int r, int b) { return 32 * j + 16 * (r >> 1) + 4 * (lane & 3) + b; }


void orc_pack_i8(const uint8_t* codes, const uint16_t* scale, const uint8_t* zero, int R, int K, int bits,
                 uint8_t* out) {
    const int NS = R / 16, NT = K / GROUP, WB = orc_tile_wbytes(bits), TB = WB + META;
    for (int s = 0; s < NS; ++s)
        for (int tt = 0; tt < NT; ++tt) {
            uint8_t* tile = out + ((size_t)s * NT + tt) * TB;
            memset(tile, 0, (size_t)TB);
            const uint8_t* c0 = codes + (size_t)(16 * s) * K + (size_t)tt * GROUP;
            for (int lane = 0; lane < 32; ++lane)
                for (int j = 0; j < 4; ++j)
                    for (int r = 0; r < 4; ++r)
                        for (int b = 0; b < 4; ++b) {
                            const uint32_t v = c0[(size_t)tile_row(lane, r) * K + tile_col(lane, j, r, b)];
                            if (bits == 8) {
                                tile[((j * 32 + lane) * 4 + r) * 4 + b] = (uint8_t)v;
                            } else if (bits == 4) {
                                const int w = 2 * j + (r >> 1), u = w >> 2;
                                uint8_t* p = tile + ((u * 32 + lane) * 4 + (w & 3)) * 4 + b;
                                *p |= (uint8_t)((v & 0xF) << (4 * (r & 1)));
                            } else {
                                uint8_t* p = tile + (lane * 4 + j) * 4 + b;
                                *p |= (uint8_t)((v & 3) << (2 * r));
                                if (bits == 3) {
                                    uint8_t* hp = tile + 512 + (lane * 2 + (j >> 1)) * 4 + b;
                                    *hp |= (uint8_t)(((v >> 2) & 1) << (4 * (j & 1) + r));
                                }
                            }
                        }
            for (int i = 0; i < 16; ++i) {
                const uint16_t sc = scale[(size_t)(16 * s + i) * NT + tt];
                memcpy(tile + WB + 2 * i, &sc, 2);
                tile[WB + 32 + i] = zero[(size_t)(16 * s + i) * NT + tt];
            }
        }
}

void orc_unpack_i8(const uint8_t* blob, int R, int K, int bits, uint8_t* codes, uint16_t* scale, uint8_t* zero) {
    const int NS = R / 16, NT = K / GROUP, WB = orc_tile_wbytes(bits), TB = WB + META;
    for (int s = 0; s < NS; ++s)
        for (int tt = 0; tt < NT; ++tt) {
            const uint8_t* tile = blob + ((size_t)s * NT + tt) * TB;
            uint8_t* c0 = codes + (size_t)(16 * s) * K + (size_t)tt * GROUP;
            for (int lane = 0; lane < 32; ++lane)
                for (int j = 0; j < 4; ++j)
                    for (int r = 0; r < 4; ++r)
                        for (int b = 0; b < 4; ++b) {
                            uint32_t v;
                            if (bits == 8) {
                                v = tile[((j * 32 + lane) * 4 + r) * 4 + b];
                            } else if (bits == 4) {
                                const int w = 2 * j + (r >> 1), u = w >> 2;
                                v = (tile[((u * 32 + lane) * 4 + (w & 3)) * 4 + b] >> (4 * (r & 1))) & 0xF;
                            } else {
                                v = (tile[(lane * 4 + j) * 4 + b] >> (2 * r)) & 3;
                                if (bits == 3)
                                    v |= ((uint32_t)(tile[512 + (lane * 2 + (j >> 1)) * 4 + b] >> (4 * (j & 1) + r)) & 1u) << 2;
                            }
                            c0[(size_t)tile_row(lane, r) * K + tile_col(lane, j, r, b)] = (uint8_t)v;
                        }
            for (int i = 0; i < 16; ++i) {
                uint16_t sc;
                memcpy(&sc, tile + WB + 2 * i, 2);
                scale[(size_t)(16 * s + i) * NT + tt] = sc;
                zero[(size_t)(16 * s + i) * NT + tt] = tile[WB + 32 + i];
            }
        }
}

/* quant/packlib.py:98-102: packed row 16 s + k is gate row 8 s + k (k < 8) or up row I + 8 s + k - 8. */
void orc_gu_row_perm(int I, int32_t* perm) {
    for (int s = 0; s < I / 8; ++s)
        for (int k = 0; k < 8; ++k) {
            perm[16 * s + k] = 8 * s + k;
            perm[16 * s + 8 + k] = I + 8 * s + k;
        }
}

/* ------------------------------------------------------------------------------------------------------------
 * A8: symmetric int8 per (row, 128-group); s = max(max|v| / 127, 1e-30), q = clamp(rint(v / s), +-127),
 * sum = sum of q. engine/ops.cu:42-66 (quant_row_smem), engine/tests/test_moe_i8.cu:52-71. Output in logical
 * column order (the reference stores a fragment permutation; the order inside a group is a layout choice).
 * ------------------------------------------------------------------------------------------------------------ */
static void quant_group_div(const float* v, int8_t* q, float* s_out, int32_t* sum_out) {
    float m = 0.0f;
    for (int i = 0; i < GROUP; ++i) m = fmaxf(m, fabsf(v[i]));
    const float s = fmaxf(m / 127.0f, 1e-30f);
    int32_t sum = 0;
    for (int i = 0; i < GROUP; ++i) {
        float r = rintf(v[i] / s);
        r = r > 127.0f ? 127.0f : r < -127.0f ? -127.0f : r;
        q[i] = (int8_t)(int)r;
        sum += (int)r;
    }
    *s_out = s;
    *sum_out = sum;
}

void orc_quant_a8(const float* x, int rows, int K, int8_t* q, float* s, int32_t* sum) {
    const int G = K / GROUP;
    for (int r = 0; r < rows; ++r)
        for (int g = 0; g < G; ++g)
            quant_group_div(x + (size_t)r * K + (size_t)g * GROUP, q + (size_t)r * K + (size_t)g * GROUP,
                            s + (size_t)r * G + g, sum + (size_t)r * G + g);
}

/* ------------------------------------------------------------------------------------------------------------
 * Router logits: logits[t, e] = sum_k x[t, k] Wr[k, e]. engine/ops.cu:137-205 splits K over 8 CTAs and
 * adds the 8 partials in a fixed order (engine/ops.cu:264-265). This build fixes the whole order: partial c
 * is an fma chain over k = c H/8 .. (c + 1) H/8 - 1 ascending from 0, and the partials are added c = 0..7
 * left to right. Wr is [H, E] (k-major), fp32.
 * ------------------------------------------------------------------------------------------------------------ */
void orc_router_logits(const float* x, const float* Wr, int T, int H, int E, float* logits) {
    const int KC = 8, KW = H / KC;
#pragma omp parallel for schedule(static)
    for (int t = 0; t < T; ++t) {
        float* part = (float*)malloc(sizeof(float) * (size_t)KC * E);
        for (int c = 0; c < KC; ++c)
            for (int e = 0; e < E; ++e) {
                float p = 0.0f;
                for (int k = c * KW; k < (c + 1) * KW; ++k) p = fmaf(x[(size_t)t * H + k], Wr[(size_t)k * E + e], p);
                part[c * E + e] = p;
            }
        for (int e = 0; e < E; ++e) {
            float l = part[e];
            for (int c = 1; c < KC; ++c) l = l + part[c * E + e];
            logits[(size_t)t * E + e] = l;
        }
        free(part);
    }
}

/* ------------------------------------------------------------------------------------------------------------
 * Routing, engine/ops.cu:256-327 and quant/s03_teacher_pass.py:132-146:
 *   score = sigmoid(logit), s = score + bias;
 *   per block of `block` tokens: pool = top-C experts by max_t s, ranked (value desc, index asc);
 *   per token: top-K of s inside the pool, (value desc, index asc);
 *   w_k = score_k / (sum_k score_k + 1e-20) * rscale, the sum taken k = 0..K-1 in rank order.
 * C >= E disables the pool (plain top-K of E). The weight uses the sigmoid score itself, as route() does.
 * ------------------------------------------------------------------------------------------------------------ */
static inline int beats(float a, int ia, float b, int ib) { return a > b || (a == b && ia < ib); }

void orc_route(const float* logits, const float* bias, int T, int E, int K, int C, int block, float rscale,
               int32_t* topk, float* topw) {
    float* sig = (float*)malloc(sizeof(float) * (size_t)T * E);
    float* s = (float*)malloc(sizeof(float) * (size_t)T * E);
    float* key = (float*)malloc(sizeof(float) * (size_t)E);
    char* inpool = (char*)malloc((size_t)E);
    char* taken = (char*)malloc((size_t)E);
    for (size_t i = 0; i < (size_t)T * E; ++i) {
        sig[i] = orc_sigmoid(logits[i]);
        s[i] = sig[i] + bias[i % (size_t)E];
    }
    for (int b0 = 0; b0 < T; b0 += block) {
        const int b1 = b0 + block < T ? b0 + block : T;
        for (int e = 0; e < E; ++e) {
            float m = -INFINITY;
            for (int t = b0; t < b1; ++t) m = fmaxf(m, s[(size_t)t * E + e]);
            key[e] = m;
        }
        for (int e = 0; e < E; ++e) {
            int rank = 0;
            for (int j = 0; j < E; ++j) rank += beats(key[j], j, key[e], e);
            inpool[e] = (C >= E) || rank < C;
        }
        for (int t = b0; t < b1; ++t) {
            const float* st = s + (size_t)t * E;
            memset(taken, 0, (size_t)E);
            float sum = 0.0f;
            for (int k = 0; k < K; ++k) {
                int best = -1;
                for (int e = 0; e < E; ++e)
                    if (inpool[e] && !taken[e] && (best < 0 || beats(st[e], e, st[best], best))) best = e;
                taken[best] = 1;
                topk[(size_t)t * K + k] = best;
                sum = sum + sig[(size_t)t * E + best];
            }
            for (int k = 0; k < K; ++k)
                topw[(size_t)t * K + k] = sig[(size_t)t * E + topk[(size_t)t * K + k]] / (sum + 1e-20f) * rscale;
        }
    }
    free(sig); free(s); free(key); free(inpool); free(taken);
}

/* ------------------------------------------------------------------------------------------------------------
 * Dispatch (engine/ops.cu:333-370, :384-423): routed slots [0, T K) grouped by expert (index ascending), inside
 * an expert by token ascending; shared slots T K + t. tok_slots is [T, K + 1]: the token's K routed slots in
 * rank order, then its shared slot (-1 without a shared expert). Returns the number of slots.
 * ------------------------------------------------------------------------------------------------------------ */
int orc_dispatch(const int32_t* topk, const float* topw, int T, int E, int K, int has_shared, int32_t* count,
                 int32_t* start, int32_t* slot_token, float* slot_weight, int32_t* tok_slots) {
    int32_t* fill = (int32_t*)malloc(sizeof(int32_t) * (size_t)E);
    for (int e = 0; e < E; ++e) count[e] = 0;
    for (int i = 0; i < T * K; ++i) count[topk[i]]++;
    int run = 0;
    for (int e = 0; e < E; ++e) { start[e] = run; fill[e] = run; run += count[e]; }
    for (int t = 0; t < T; ++t)
        for (int k = 0; k < K; ++k) {
            const int e = topk[(size_t)t * K + k], sl = fill[e]++;
            slot_token[sl] = t;
            slot_weight[sl] = topw[(size_t)t * K + k];
            tok_slots[(size_t)t * (K + 1) + k] = sl;
        }
    for (int t = 0; t < T; ++t) {
        if (has_shared) {
            slot_token[T * K + t] = t;
            slot_weight[T * K + t] = 1.0f;
        }
        tok_slots[(size_t)t * (K + 1) + K] = has_shared ? T * K + t : -1;
    }
    free(fill);
    return T * K + (has_shared ? T : 0);
}

/* ------------------------------------------------------------------------------------------------------------
 * Expert integer core, engine/moe_i8.cu:1-14, :364-376:
 *   P[r, g] = sum_{k in group g} code[r, k] * xq[k]  -  zero[r, g] * xsum[g]        (exact int32)
 * ------------------------------------------------------------------------------------------------------------ */
void orc_group_products(const uint8_t* codes, const uint8_t* zero, int R, int K, const int8_t* xq,
                        const int32_t* xsum, int32_t* P) {
    const int G = K / GROUP;
    for (int r = 0; r < R; ++r)
        for (int g = 0; g < G; ++g) {
            const uint8_t* c = codes + (size_t)r * K + (size_t)g * GROUP;
            const int8_t* a = xq + (size_t)g * GROUP;
            int32_t acc = 0;
            for (int k = 0; k < GROUP; ++k) acc += (int32_t)c[k] * (int32_t)a[k];
            P[(size_t)r * G + g] = acc - (int32_t)zero[(size_t)r * G + g] * xsum[g];
        }
}

/* fp32 epilogue of one row, engine/moe_i8.cu:377-383: one accumulator per (row, token), starting at 0, and
 * for g ascending  acc = fma(scale_w[r, g] * scale_x[g], float(P[r, g]), acc)  -- the same operation sequence
 * on CPU and GPU (the product of the two scales rounded to fp32, then one fused multiply-add per group). */
static inline float row_epilogue(const int32_t* P, const uint16_t* sw, const float* sx, int G) {
    float acc = 0.0f;
    for (int g = 0; g < G; ++g) acc = fmaf(orc_f16_to_f32(sw[g]) * sx[g], (float)P[g], acc);
    return acc;
}

/* FWHT-512 in fp32, Sylvester order: stages h = 1, 2, ..., 256, butterfly (a, b) -> (a + b, a - b) on indices
 * (j, j + h), j & h == 0 (engine/moe_i8.cu:462-475), then scaled by 1/sqrt(512) (:478). */
void orc_fwht512_f32(float* v) {
    for (int h = 1; h < 512; h <<= 1)
        for (int j = 0; j < 512; ++j)
            if (!(j & h)) {
                const float a = v[j], b = v[j + h];
                v[j] = a + b;
                v[j + h] = a - b;
            }
    for (int j = 0; j < 512; ++j) v[j] = v[j] * 0.04419417382415922f;
}

/* Z' = A8(Z H512 / sqrt(512)) per slot, engine/moe_i8.cu:447-502: the group quantiser multiplies by the
 * reciprocal of the scale (q = rint(v * (1/s))), unlike the activation quantiser. Logical order out. */
static void fwht_a8_one(const uint16_t* z, int8_t* q, float* s, int32_t* sum) {
    float v[512];
    for (int j = 0; j < 512; ++j) v[j] = orc_f16_to_f32(z[j]);
    orc_fwht512_f32(v);
    for (int g = 0; g < 4; ++g) {
        const float* vg = v + g * GROUP;
        float m = 0.0f;
        for (int i = 0; i < GROUP; ++i) m = fmaxf(m, fabsf(vg[i]));
        const float sc = fmaxf(m / 127.0f, 1e-30f), inv = 1.0f / sc;
        int32_t acc = 0;
        for (int i = 0; i < GROUP; ++i) {
            float r = rintf(vg[i] * inv);
            r = r > 127.0f ? 127.0f : r < -127.0f ? -127.0f : r;
            q[g * GROUP + i] = (int8_t)(int)r;
            acc += (int)r;
        }
        s[g] = sc;
        sum[g] = acc;
    }
}

void orc_fwht_a8(const uint16_t* Z, int nslots, int8_t* q, float* s, int32_t* sum) {
#pragma omp parallel for schedule(static)
    for (int i = 0; i < nslots; ++i) fwht_a8_one(Z + (size_t)i * 512, q + (size_t)i * 512, s + (size_t)i * 4, sum + (size_t)i * 4);
}

/* one expert's unpacked matrices */
typedef struct {
    uint8_t *gu_c, *gu_z, *d_c, *d_z;
    uint16_t *gu_s, *d_s;
} unpacked;

static int unpack_expert(const orc_layer* L, int e, unpacked* u) {
    const int b = L->bits[e];
    if (orc_tile_wbytes(b) < 0) return -1;
    orc_unpack_i8(L->blob + L->gu_off[e], 2 * L->I, L->H, b, u->gu_c, u->gu_s, u->gu_z);
    orc_unpack_i8(L->blob + L->d_off[e], L->H, L->I, b, u->d_c, u->d_s, u->d_z);
    return 0;
}

static int alloc_unpacked(const orc_layer* L, unpacked* u) {
    const size_t ngu = (size_t)2 * L->I * L->H, nd = (size_t)L->H * L->I;
    u->gu_c = (uint8_t*)malloc(ngu);
    u->gu_z = (uint8_t*)malloc(ngu / GROUP);
    u->gu_s = (uint16_t*)malloc(2 * ngu / GROUP);
    u->d_c = (uint8_t*)malloc(nd);
    u->d_z = (uint8_t*)malloc(nd / GROUP);
    u->d_s = (uint16_t*)malloc(2 * nd / GROUP);
    return (u->gu_c && u->gu_z && u->gu_s && u->d_c && u->d_z && u->d_s) ? 0 : -1;
}

static void free_unpacked(unpacked* u) {
    free(u->gu_c); free(u->gu_z); free(u->gu_s); free(u->d_c); free(u->d_z); free(u->d_s);
}

/* zin != NULL: the gate_up outputs Z of every slot are given (gate_up is skipped; xq, xs, xsum unused) */
static int experts_impl(const orc_layer* L, const int8_t* xq, const float* xs, const int32_t* xsum,
                        const uint16_t* zin, int yhalf, int T, const int32_t* count, const int32_t* start,
                        const int32_t* slot_token, const float* slot_weight, const int32_t* tok_slots, uint16_t* Z,
                        int8_t* zq, float* zs, int32_t* zsum, float* Y, float* out, int nthreads) {
    const int H = L->H, I = L->I, E = L->E, K = L->K, GH = H / GROUP, GI = I / GROUP;
    const int nexp = E + (L->has_shared ? 1 : 0);
    const int S = T * K + (L->has_shared ? T : 0);
    if (I != 512 || H % GROUP) return -2;
    for (int e = 0; e < nexp; ++e)
        if (orc_tile_wbytes(L->bits[e]) < 0) return -3;
    float* Yw = Y ? Y : (float*)malloc(sizeof(float) * (size_t)S * H);
    int err = 0;
#ifdef _OPENMP
    if (nthreads <= 0) nthreads = omp_get_max_threads();
#else
    (void)nthreads;
#endif
#pragma omp parallel num_threads(nthreads) reduction(| : err)
    {
        unpacked u;
        if (alloc_unpacked(L, &u)) err |= 1;
        int32_t* P = (int32_t*)malloc(sizeof(int32_t) * (size_t)2 * I * GH);
        int32_t* perm = (int32_t*)malloc(sizeof(int32_t) * (size_t)2 * I);
        float* gacc = (float*)malloc(sizeof(float) * (size_t)2 * I);
        uint16_t zrow[512];
        int8_t qrow[512];
        float srow[4];
        int32_t sumrow[4];
        orc_gu_row_perm(I, perm);
#pragma omp for schedule(dynamic, 1)
        for (int e = 0; e < nexp; ++e) {
            const int n = e < E ? count[e] : T;
            const int s0 = e < E ? start[e] : T * K;
            if (n == 0 || err) continue;
            unpack_expert(L, e, &u);
            for (int i = 0; i < n; ++i) {
                const int slot = s0 + i, tok = slot_token[slot];
                if (zin) {
                    memcpy(zrow, zin + (size_t)slot * I, sizeof(zrow));
                } else {
                    /* gate_up: packed rows -> logical rows (gate 0..I-1, up I..2I-1) */
                    orc_group_products(u.gu_c, u.gu_z, 2 * I, H, xq + (size_t)tok * H, xsum + (size_t)tok * GH, P);
                    for (int p = 0; p < 2 * I; ++p)
                        gacc[perm[p]] = row_epilogue(P + (size_t)p * GH, u.gu_s + (size_t)p * GH, xs + (size_t)tok * GH,
                                                     GH);
                    for (int j = 0; j < I; ++j) zrow[j] = orc_f32_to_f16(orc_silu(gacc[j]) * gacc[I + j]);
                }
                fwht_a8_one(zrow, qrow, srow, sumrow);
                if (Z) memcpy(Z + (size_t)slot * I, zrow, sizeof(zrow));
                if (zq) memcpy(zq + (size_t)slot * I, qrow, sizeof(qrow));
                if (zs) memcpy(zs + (size_t)slot * 4, srow, sizeof(srow));
                if (zsum) memcpy(zsum + (size_t)slot * 4, sumrow, sizeof(sumrow));
                /* down: Y[slot, h] = w_slot * acc_h */
                orc_group_products(u.d_c, u.d_z, H, I, qrow, sumrow, P);
                const float w = slot_weight[slot];
                for (int h = 0; h < H; ++h) {
                    const float y = w * row_epilogue(P + (size_t)h * GI, u.d_s + (size_t)h * GI, srow, GI);
                    /* yhalf: the build's fast-numerics slot outputs, rounded to fp16 (nearest even) */
                    Yw[(size_t)slot * H + h] = yhalf ? orc_f16_to_f32(orc_f32_to_f16(y)) : y;
                }
            }
        }
        free(P); free(perm); free(gacc);
        free_unpacked(&u);
    }
    if (!err) {
        const int KK = K + (L->has_shared ? 1 : 0);
#pragma omp parallel for schedule(static) num_threads(nthreads)
        for (int t = 0; t < T; ++t)
            for (int h = 0; h < H; ++h) {
                float acc = 0.0f;
                for (int k = 0; k < KK; ++k) acc = acc + Yw[(size_t)tok_slots[(size_t)t * (K + 1) + k] * H + h];
                out[(size_t)t * H + h] = acc;
            }
    }
    if (!Y) free(Yw);
    return err ? -1 : 0;
}

int orc_experts(const orc_layer* L, const int8_t* xq, const float* xs, const int32_t* xsum, int T,
                const int32_t* count, const int32_t* start, const int32_t* slot_token, const float* slot_weight,
                const int32_t* tok_slots, uint16_t* Z, int8_t* zq, float* zs, int32_t* zsum, float* Y, float* out,
                int nthreads) {
    return experts_impl(L, xq, xs, xsum, NULL, 0, T, count, start, slot_token, slot_weight, tok_slots, Z, zq, zs, zsum, Y,
                        out, nthreads);
}

int orc_experts_from_z(const orc_layer* L, const uint16_t* Z, int yhalf, int T, const int32_t* count,
                       const int32_t* start, const int32_t* slot_token, const float* slot_weight,
                       const int32_t* tok_slots, int8_t* zq, float* zs, int32_t* zsum, float* Y, float* out,
                       int nthreads) {
    return experts_impl(L, NULL, NULL, NULL, Z, yhalf, T, count, start, slot_token, slot_weight, tok_slots, NULL, zq, zs,
                        zsum, Y, out, nthreads);
}

/* ------------------------------------------------------------------------------------------------------------
 * fp64 dequantise-then-matmul, engine/tests/gen_moe_case.py:77-93 with its helpers :20-36:
 *   x' = a8(x) (dequantised, fp32), h = W_gu x' , z = fp16(SiLU(h_g) h_u), z' = a8(z H512) (fp32),
 *   acc += w * (W_d z').   Matrix products and the Hadamard transform in fp64.
 * ------------------------------------------------------------------------------------------------------------ */
static void a8_dequant(const float* v, int n, float* out) {
    for (int g = 0; g < n / GROUP; ++g) {
        int8_t q[GROUP];
        float s;
        int32_t sum;
        quant_group_div(v + g * GROUP, q, &s, &sum);
        for (int i = 0; i < GROUP; ++i) out[g * GROUP + i] = (float)q[i] * s;
    }
}

int orc_reference_f64(const orc_layer* L, const float* x, int T, const int32_t* topk, const float* topw,
                      double* out, int nthreads) {
    const int H = L->H, I = L->I, E = L->E, K = L->K, GH = H / GROUP, GI = I / GROUP;
    const int nexp = E + (L->has_shared ? 1 : 0);
    if (I != 512) return -2;
    for (int e = 0; e < nexp; ++e)
        if (orc_tile_wbytes(L->bits[e]) < 0) return -3;
    float* xd = (float*)malloc(sizeof(float) * (size_t)T * H);
    for (int t = 0; t < T; ++t) a8_dequant(x + (size_t)t * H, H, xd + (size_t)t * H);
    memset(out, 0, sizeof(double) * (size_t)T * H);
    /* per-expert contribution, accumulated per token in a per-thread buffer then reduced in expert order */
    double* contrib = (double*)calloc((size_t)T * (K + 1) * H, sizeof(double));
    int err = 0;
#ifdef _OPENMP
    if (nthreads <= 0) nthreads = omp_get_max_threads();
#else
    (void)nthreads;
#endif
#pragma omp parallel num_threads(nthreads) reduction(| : err)
    {
        unpacked u;
        if (alloc_unpacked(L, &u)) err |= 1;
        int32_t* perm = (int32_t*)malloc(sizeof(int32_t) * (size_t)2 * I);
        double* Wgu = (double*)malloc(sizeof(double) * (size_t)2 * I * H);
        double* Wd = (double*)malloc(sizeof(double) * (size_t)H * I);
        double h[1024];
        float zf[512], za[512];
        orc_gu_row_perm(I, perm);
#pragma omp for schedule(dynamic, 1)
        for (int e = 0; e < nexp; ++e) {
            int used = 0;
            for (int i = 0; i < T * K && !used; ++i) used = (e == E) || topk[i] == e;
            if (!used || err || I * 2 > 1024) continue;
            unpack_expert(L, e, &u);
            for (int p = 0; p < 2 * I; ++p)
                for (int k = 0; k < H; ++k)
                    Wgu[(size_t)perm[p] * H + k] = ((double)u.gu_c[(size_t)p * H + k] - (double)u.gu_z[(size_t)p * GH + k / GROUP]) *
                                                   (double)orc_f16_to_f32(u.gu_s[(size_t)p * GH + k / GROUP]);
            for (int r = 0; r < H; ++r)
                for (int k = 0; k < I; ++k)
                    Wd[(size_t)r * I + k] = ((double)u.d_c[(size_t)r * I + k] - (double)u.d_z[(size_t)r * GI + k / GROUP]) *
                                            (double)orc_f16_to_f32(u.d_s[(size_t)r * GI + k / GROUP]);
            for (int t = 0; t < T; ++t)
                for (int k = 0; k <= K; ++k) {
                    double w;
                    if (k < K) { if (topk[(size_t)t * K + k] != e) continue; w = topw[(size_t)t * K + k]; }
                    else { if (e != E) continue; w = 1.0; }
                    const float* xt = xd + (size_t)t * H;
                    for (int r = 0; r < 2 * I; ++r) {
                        double a = 0.0;
                        for (int c = 0; c < H; ++c) a += Wgu[(size_t)r * H + c] * (double)xt[c];
                        h[r] = a;
                    }
                    double zd[512];
                    for (int j = 0; j < I; ++j) {
                        const double g = h[j];
                        const float zz = (float)(g / (1.0 + exp(-g)) * h[I + j]);
                        zd[j] = (double)orc_f16_to_f32(orc_f32_to_f16(zz));
                    }
                    for (int hh = 1; hh < 512; hh <<= 1)
                        for (int j = 0; j < 512; ++j)
                            if (!(j & hh)) { const double a = zd[j], b = zd[j + hh]; zd[j] = a + b; zd[j + hh] = a - b; }
                    for (int j = 0; j < 512; ++j) zf[j] = (float)(zd[j] / sqrt(512.0));
                    a8_dequant(zf, 512, za);
                    double* o = contrib + ((size_t)t * (K + 1) + k) * H;
                    for (int r = 0; r < H; ++r) {
                        double a = 0.0;
                        for (int c = 0; c < I; ++c) a += Wd[(size_t)r * I + c] * (double)za[c];
                        o[r] = w * a;
                    }
                }
        }
        free(perm); free(Wgu); free(Wd);
        free_unpacked(&u);
    }
    for (int t = 0; t < T; ++t)
        for (int k = 0; k <= K; ++k)
            for (int r = 0; r < H; ++r) out[(size_t)t * H + r] += contrib[((size_t)t * (K + 1) + k) * H + r];
    free(contrib);
    free(xd);
    return err ? -1 : 0;
}

/* ---- combine + un-rotation + residual + next-layer norm / rotation / A8 (engine/ops.cu:507-549) ---------------
 * Unnormalised Sylvester FWHT of n values, stages h = 1, 2, ..., n/2 ascending (engine/ops.cu:458-474 and the
 * bits 8-10 stages of :477-505 run in the same ascending order). */
/* Dense W.A8 projection (engine/engine.cu:380-383, :425, :434): one matrix, every token, the same integer core
 * and fp32 epilogue as the experts (orc_group_products, row_epilogue); accumulate adds to y (fp32 add). */
int orc_dense(const uint8_t* blob, int R, int K, int bits, const int8_t* xq, const float* xs, const int32_t* xsum,
              int T, float* y, int accumulate, int nthreads) {
    if (orc_tile_wbytes(bits) < 0 || R % 16 || K % GROUP) return -1;
    const int G = K / GROUP;
    uint8_t* c = (uint8_t*)malloc((size_t)R * K);
    uint8_t* z = (uint8_t*)malloc((size_t)R * G);
    uint16_t* s = (uint16_t*)malloc(sizeof(uint16_t) * (size_t)R * G);
    if (!c || !z || !s) { free(c); free(z); free(s); return -2; }
    orc_unpack_i8(blob, R, K, bits, c, s, z);
#ifdef _OPENMP
    if (nthreads <= 0) nthreads = omp_get_max_threads();
#else
    (void)nthreads;
#endif
    int err = 0;
#pragma omp parallel num_threads(nthreads) reduction(| : err)
    {
        int32_t* P = (int32_t*)malloc(sizeof(int32_t) * (size_t)R * G);
        if (!P) err |= 1;
#pragma omp for schedule(static)
        for (int t = 0; t < T; ++t) {
            if (!P) continue;
            orc_group_products(c, z, R, K, xq + (size_t)t * K, xsum + (size_t)t * G, P);
            for (int r = 0; r < R; ++r) {
                const float v = row_epilogue(P + (size_t)r * G, s + (size_t)r * G, xs + (size_t)t * G, G);
                float* yo = y + (size_t)t * R + r;
                *yo = accumulate ? *yo + v : v;
            }
        }
        free(P);
    }
    free(c); free(z); free(s);
    return err ? -2 : 0;
}

static void fwht_n(float* v, int n) {
    for (int h = 1; h < n; h <<= 1)
        for (int j = 0; j < n; ++j)
            if (!(j & h)) {
                const float a = v[j], b = v[j + h];
                v[j] = a + b;
                v[j + h] = a - b;
            }
}

#define INV_SQRT_2048 0.02209708691207961f

/* Per token t (H = 2048):
 *   x = sum_k Y[tok_slots[t, k]] (k = 0 .. nk-1 ascending, from 0)                       engine/ops.cu:515-520
 *   h[t] = h[t] + (FWHT(x) * signs) * 2048^-1/2                                          :521-535 (un-rotation)
 *   r = 1 / sqrt(sum(h[t]^2) / 2048 + eps); y = FWHT((h[t] * r) * signs) * 2048^-1/2     :74-114 (norm_rot_body)
 *   (q, s, sum) = A8(y)                                                                   :40-66
 * The sum of squares follows the GPU's tree: thread i (0 .. 255) adds h[i + 256 j]^2 for j = 0 .. 7 in order,
 * a 64-lane xor butterfly (1, 2, .., 32) sums each wave, and the 4 wave sums are added in order. */
void orc_combine_norm(const float* Y, const int32_t* tok_slots, int T, int nk, int K1, const float* signs, float eps,
                      float* h, int8_t* q, float* s, int32_t* sum) {
    enum { H = 2048 };
#pragma omp parallel for schedule(static)
    for (int t = 0; t < T; ++t) {
        float x[H], part[256];
        for (int c = 0; c < H; ++c) x[c] = 0.0f;
        for (int k = 0; k < nk; ++k) {
            const float* y = Y + (size_t)tok_slots[(size_t)t * K1 + k] * H;
            for (int c = 0; c < H; ++c) x[c] = x[c] + y[c];
        }
        fwht_n(x, H);
        float* hr = h + (size_t)t * H;
        for (int c = 0; c < H; ++c) hr[c] = hr[c] + (x[c] * signs[c]) * INV_SQRT_2048;
        for (int i = 0; i < 256; ++i) {
            float p = 0.0f;
            for (int j = 0; j < 8; ++j) p = p + hr[i + 256 * j] * hr[i + 256 * j];
            part[i] = p;
        }
        float tot = 0.0f;
        for (int w = 0; w < 4; ++w) {
            float a[64], b[64];
            for (int l = 0; l < 64; ++l) a[l] = part[64 * w + l];
            for (int o = 1; o < 64; o <<= 1) {
                for (int l = 0; l < 64; ++l) b[l] = a[l] + a[l ^ o];
                for (int l = 0; l < 64; ++l) a[l] = b[l];
            }
            tot = w == 0 ? a[0] : tot + a[0];
        }
        const float r = 1.0f / sqrtf(tot / 2048.0f + eps);
        for (int c = 0; c < H; ++c) x[c] = (hr[c] * r) * signs[c];
        fwht_n(x, H);
        for (int c = 0; c < H; ++c) x[c] = x[c] * INV_SQRT_2048;
        for (int g = 0; g < H / GROUP; ++g)
            quant_group_div(x + g * GROUP, q + (size_t)t * H + g * GROUP, s + (size_t)t * (H / GROUP) + g,
                            sum + (size_t)t * (H / GROUP) + g);
    }
}
