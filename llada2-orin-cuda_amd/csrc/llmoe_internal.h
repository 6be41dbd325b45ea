// Internal declarations shared by the libllmoe translation units: device data formats, numeric helpers that
// must match the CPU checker bit for bit, and the host-side launchers each kernel file exports.
#pragma once
#include <hip/hip_runtime.h>
#include <cstddef>
#include <cstdint>

namespace llmoe {

constexpr int GROUP = 128;       // quantisation group along K (weights and activations)
constexpr int SB_K = 512;        // K columns per superblock = 4 groups
constexpr int META_SB = 192;     // per strip and superblock: 64 fp16 scales + 64 u8 zeros
constexpr int ROUTER_KC = 8;     // router K chunks (fixed summation order)

// One work unit of the expert GEMMs: `ntok` consecutive slots of one expert, row block `rb` of its matrix.
struct Item {
    int expert;
    int slot0;
    int ntok;
    int rb;
};

// GEMM geometry shared by the dispatch kernels (which emit the work units) and the GEMM kernels: a workgroup of
// GEMM_WAVES waves covers 16 * GEMM_WAVES * spw rows, spw = strips per wave chosen by code width so that every
// wave streams about the same bytes (2-bit codes: 4 strips of gate_up, 3/4-bit: 2, 8-bit: 1; down has K/4 and
// four times the strips).
constexpr int GEMM_WAVES = 4;
__host__ __device__ constexpr int gemm_spw(bool down, int bits) {
    return (down ? 4 : 1) * (bits == 2 ? 4 : bits == 8 ? 1 : 2);
}
// row blocks (work units per work item) of a gate_up [2I = 1024] or down [H = 2048] matrix
__host__ __device__ constexpr int gemm_row_blocks(bool down, int bits) {
    return (down ? 2048 : 1024) / (16 * GEMM_WAVES * gemm_spw(down, bits));
}
constexpr int MAX_UNITS_PER_ITEM = 16;   // gemm_row_blocks(false, 8)

// Tiled GEMM (experts with many tokens): a work unit is a chunk of <= TILED_NTOK slots of one expert and a
// range of row blocks (Item.rb = first | count << 16); the workgroup stages the chunk's activations in LDS once
// and its tiled_waves waves stream tiled_spw strips each per row block. An expert takes tiled units when it has
// more than TILED_MIN slots, otherwise streamed units of 16 slots.
// K = 2048 (gate_up, dense): 8 waves of 2 strips (1 for 8-bit codes). K = 512 (down): 16 waves of 1 strip, whose
// registers fit 4 waves per SIMD (the vector issue rate per SIMD grows with the waves it can pick from).
constexpr int TILED_NTOK = 64;
constexpr int TILED_MIN = 16;
__host__ __device__ constexpr int tiled_waves(bool down) { return down ? 16 : 8; }
__host__ __device__ constexpr int tiled_spw(bool down, int bits) { return down ? 1 : bits == 8 ? 1 : 2; }
__host__ __device__ constexpr int tiled_row_blocks(bool down, int bits) {
    return (down ? 2048 : 1024) / (16 * tiled_waves(down) * tiled_spw(down, bits));
}
// chunks of an expert with c slots: n = ceil(c / TILED_NTOK) chunks of `per` slots (a multiple of 16), the last
// one shorter
__host__ __device__ constexpr int tiled_chunks(int c) { return (c + TILED_NTOK - 1) / TILED_NTOK; }
__host__ __device__ constexpr int tiled_per(int c) {
    return c <= 0 ? 0 : (((c + tiled_chunks(c) - 1) / tiled_chunks(c)) + 15) / 16 * 16;
}
// Tiled work partition (per GEMM): the chunks are listed in order, chunk i spanning positions
// [pre_i, pre_i + s + nrb_i c_i) with s the cost of staging its activations and c_i the estimated cost of one of its
// nrb_i row-block tasks (by code width and 16-slot tiles), row block r starting at pre_i + s + r c_i. Workgroup w of the G-workgroup grid runs the tasks whose
// start lies in [ceil(w C / G), ceil((w + 1) C / G)), C = the total; tstart[w] = its first task as
// chunk | rb << TASK_RB_SHIFT (tstart[G] = all chunks, rb 0).
constexpr int TASK_RB_SHIFT = 20;

// Device weight layout (written by relayout_matrix from packlib "i8"):
//   matrix [R, K] = R/16 strips of 16 rows; a strip = K/512 superblocks; a superblock (4 groups of 128) =
//     BITS x 1024 B of codes: load i of lane l (64 lanes) at i*1024 + 16 l (one dwordx4 per lane and load)
//     128 B scales  [q 4][tile 4][v 4] fp16      (lane quad q = l/16 reads 32 B at 32 q)
//      64 B zeros   [q 4][tile 4][v 4] u8        (lane quad q reads 16 B at 128 + 16 q)
//   so one superblock has the same byte count as 4 packlib tiles (4 (256 BITS + 48)).
// Lane l of the MFMA A operand holds strip row l%16 and, for the group's two 64-column halves h, columns
//   64 h + 16 (l/16) + 0..15; output row 4 (l/16) + v of v_mfma_i32_16x16x64_i8 is strip row 4 (l/16) + v.
// gate_up strips are stored in the row order gate j, up j, gate j+1, up j+1 per lane quad, so each lane ends
// with the gate and up accumulators of the same intermediate channels (see relayout.hip).
__host__ __device__ constexpr size_t sb_bytes(int bits) { return size_t(bits) * 1024 + META_SB; }
__host__ __device__ constexpr size_t matrix_dev_bytes(int R, int K, int bits) {
    return size_t(R / 16) * size_t(K / SB_K) * sb_bytes(bits);
}

// ---- numerics shared with the CPU checker (same fp32 operation sequence, compiled with fp-contract off) ----

__device__ __forceinline__ float pow2i(int k) { return __int_as_float((k + 127) << 23); }

// exp(x): Cody-Waite reduction with ln2 = hi + lo (hi has 12 trailing zero bits), Taylor polynomial of degree 7
// on |r| <= ln2/2, scaling by 2^n as two exact power-of-two factors.
// exp's polynomial path (Cody-Waite reduction with ln2 = hi + lo, hi with 12 trailing zero bits; Taylor
// polynomial of degree 7; the 2^n scaling split in two so that n down to -150 stays exact)
__device__ __forceinline__ float exp_poly(float x) {
    const float n = __builtin_rintf(x * 1.44269502162933349609375f);
    float r = __builtin_fmaf(n, -0.693145751953125f, x);
    r = __builtin_fmaf(n, -1.428606765330187045037746429443359375e-06f, r);
    float p = 1.98412701138295233249664306640625e-04f;
    p = __builtin_fmaf(p, r, 1.38888892345130443572998046875e-03f);
    p = __builtin_fmaf(p, r, 8.33333376795053482055664062500e-03f);
    p = __builtin_fmaf(p, r, 4.16666679084300994873046875000e-02f);
    p = __builtin_fmaf(p, r, 1.66666671633720397949218750000e-01f);
    p = __builtin_fmaf(p, r, 0.5f);
    p = __builtin_fmaf(p, r, 1.0f);
    p = __builtin_fmaf(p, r, 1.0f);
    const int ni = int(n), e1 = ni / 2, e2 = ni - e1;
    return (p * pow2i(e1)) * pow2i(e2);
}
__device__ __forceinline__ float exp_f32(float x) {
    // when every active lane is inside the polynomial's range (the common case) the special cases are skipped;
    // otherwise the polynomial runs on x clamped into the range and the special results are selected. Either
    // way the values equal those of the early-return form of the CPU checker.
    const bool in = x >= -103.97208404541016f && x <= 88.72283935546875f;   // false for nan
    if (__all(in)) return exp_poly(x);
    float v = exp_poly(fminf(fmaxf(x, -103.97208404541016f), 88.72283935546875f));
    v = x > 88.72283935546875f ? __builtin_inff() : v;
    v = x < -103.97208404541016f ? 0.0f : v;
    return x != x ? x : v;
}
__device__ __forceinline__ float sigmoid_f32(float x) { return 1.0f / (1.0f + exp_f32(-x)); }
// SiLU of the gate_up epilogue, whose result is multiplied by u and rounded to fp16 (2^-11): exp(-g) by a
// Cody-Waite reduction with one ln2 constant and a degree-5 Taylor polynomial (relative error < 1e-5), scaled
// exactly by ldexp; 1 / (1 + e) by three Newton steps from a bit-pattern seed. The exp argument is clamped to
// [-104, 80] (beyond it the fp16 product no longer changes), which keeps every step finite. IEEE fma / mul / add /
// rint / min / max / ldexp only, the same sequence as the CPU checker's orc_silu.
__device__ __forceinline__ float silu_f32(float g) {
    const float x = fminf(fmaxf(-g, -104.0f), 80.0f);
    const float n = __builtin_rintf(x * 1.44269502162933349609375f);
    const float r = __builtin_fmaf(n, -0.693147182464599609375f, x);
    float p = 8.33333376795053482055664062500e-03f;
    p = __builtin_fmaf(p, r, 4.16666679084300994873046875000e-02f);
    p = __builtin_fmaf(p, r, 1.66666671633720397949218750000e-01f);
    p = __builtin_fmaf(p, r, 0.5f);
    p = __builtin_fmaf(p, r, 1.0f);
    p = __builtin_fmaf(p, r, 1.0f);
    const float d = 1.0f + __builtin_ldexpf(p, int(n));
    float q = __int_as_float(0x7EF311C3 - __float_as_int(d));
#pragma unroll
    for (int i = 0; i < 3; ++i) q = __builtin_fmaf(q, __builtin_fmaf(-d, q, 1.0f), q);
    return g * q;
}

// fp32 -> fp16 with round-to-nearest-even, spelled out in integer ops: the definition the CPU checker restates
// (orc_f32_to_f16). The kernels use the hardware conversion below; llmoe_selftest_f16 checks on the device that the
// two agree on every finite fp32 input.
__device__ __forceinline__ uint16_t f32_to_f16_bits(float f) {
    const uint32_t x = __float_as_uint(f);
    const uint32_t sign = (x >> 16) & 0x8000u, ax = x & 0x7fffffffu;
    // normal half: round the 13 dropped mantissa bits to nearest even by adding 0xFFF plus the kept lsb (a carry
    // runs into the exponent as it should), then rebias the exponent
    const uint32_t hn = ((ax + 0xFFFu + ((ax >> 13) & 1u)) >> 13) - (112u << 10);
    // every active lane a normal half (the common case): done; otherwise every range's result is computed and
    // the one for ax selected
    if (__all(ax - 0x38800000u < 0x477ff000u - 0x38800000u)) return uint16_t(sign | hn);
    // subnormal half: exact scale by 2^24 (the operand clamped so that no lane converts an inf or nan)
    const uint32_t hs = uint32_t(__builtin_rintf(__uint_as_float(ax < 0x38800000u ? ax : 0x38800000u) * 16777216.0f));
    uint32_t h = ax < 0x38800000u ? hs : hn;
    h = ax >= 0x477ff000u ? 0x7c00u : h;                                          // >= 65520 rounds to inf
    h = ax >= 0x7f800000u ? (0x7c00u | (ax > 0x7f800000u ? 0x200u : 0u)) : h;    // inf / nan
    return uint16_t(sign | h);
}

// fp32 -> fp16, round to nearest even, by v_cvt_f16_f32 (the default rounding mode): one instruction, and the same
// bits as f32_to_f16_bits for every finite input (an exhaustive sweep over the 2^32 patterns, llmoe_selftest_f16);
// a NaN input gives a NaN. The fp32 value is made opaque first: otherwise the compiler folds a preceding multiply
// into v_fma_mixlo_f16, which rounds the exact product to fp16 once instead of rounding to fp32 and then to fp16.
__device__ __forceinline__ uint16_t f32_to_f16_rne(float f) {
    asm("" : "+v"(f));
    return __builtin_bit_cast(uint16_t, static_cast<_Float16>(f));
}

// int32 -> fp32 through the MFMA accumulator: a product that starts from I2F_BIAS (the bits of 1.5 * 2^23) ends as
// the bits of the float 1.5 * 2^23 + P exactly when |P| < 2^22 (every group product: |c - z| <= 255, |xq| <= 127,
// 128 terms), so one subtraction -- cheaper than v_cvt_f32_i32 on gfx950 -- returns float(P) exactly.
constexpr int I2F_BIAS = 0x4B400000;
__device__ __forceinline__ float biased_to_f32(int c) { return __int_as_float(c) - 12582912.0f; }

// The value of lane (lane ^ o), o a wave-uniform power of two below 64 (all lanes active): DPP quad permutes for
// o = 1, 2 (no LDS round trip), ds_swizzle's xor mode inside 32-lane halves for o = 4 .. 16, ds_bpermute for
// o = 32. The same data movement as __shfl_xor.
__device__ __forceinline__ int xor_lane(int v, int o) {
    if (o == 1) return __builtin_amdgcn_mov_dpp(v, 0xB1, 0xF, 0xF, false);    // quad_perm [1, 0, 3, 2]
    if (o == 2) return __builtin_amdgcn_mov_dpp(v, 0x4E, 0xF, 0xF, false);    // quad_perm [2, 3, 0, 1]
    if (o == 4) return __builtin_amdgcn_ds_swizzle(v, (4 << 10) | 0x1F);     // and 0x1F, or 0, xor 4
    if (o == 8) return __builtin_amdgcn_ds_swizzle(v, (8 << 10) | 0x1F);
    if (o == 16) return __builtin_amdgcn_ds_swizzle(v, (16 << 10) | 0x1F);
    return __shfl_xor(v, o);
}
__device__ __forceinline__ float xor_lane(float v, int o) { return __int_as_float(xor_lane(__float_as_int(v), o)); }

// Inclusive prefix sum over the 64 lanes of a wave (all lanes active): Hillis-Steele inside each 16-lane row by
// DPP row shifts (lanes shifted in from outside the row add 0), then the totals of rows 0 and 2 added to rows 1
// and 3 (row_bcast:15), and the total of rows 0-1 added to rows 2-3 (row_bcast:31).
__device__ __forceinline__ uint32_t wave_incl_scan(uint32_t v) {
    int x = int(v);
    x += __builtin_amdgcn_update_dpp(0, x, 0x111, 0xF, 0xF, false);   // row_shr:1
    x += __builtin_amdgcn_update_dpp(0, x, 0x112, 0xF, 0xF, false);   // row_shr:2
    x += __builtin_amdgcn_update_dpp(0, x, 0x114, 0xF, 0xF, false);   // row_shr:4
    x += __builtin_amdgcn_update_dpp(0, x, 0x118, 0xF, 0xF, false);   // row_shr:8
    x += __builtin_amdgcn_update_dpp(0, x, 0x142, 0xA, 0xF, false);   // row_bcast:15 into rows 1, 3
    x += __builtin_amdgcn_update_dpp(0, x, 0x143, 0xC, 0xF, false);   // row_bcast:31 into rows 2, 3
    return uint32_t(x);
}
__device__ __forceinline__ int wave_incl_scan(int v) { return int(wave_incl_scan(uint32_t(v))); }
// 64-bit values whose sums carry nothing from bit 31 into bit 32 (fields of 16 bits): the halves scan apart
__device__ __forceinline__ uint64_t wave_incl_scan(uint64_t v) {
    return (uint64_t(wave_incl_scan(uint32_t(v >> 32))) << 32) | wave_incl_scan(uint32_t(v));
}

// The gate_up output fp16(SiLU(g) u) with the hardware transcendentals (v_exp_f32, v_rcp_f32) and conversion
// (v_cvt_f16_f32): the precision of the reference's own __expf / __fdividef / __float2half (engine/moe_i8.cu:221),
// within the fp32-stage tolerance, not bit-identical to silu_f32.
__device__ __forceinline__ uint16_t silu_mul_f16_fast(float g, float u) {
    const float e = __builtin_amdgcn_exp2f(g * -1.44269504088896341f);
    const float y = (g * __builtin_amdgcn_rcpf(1.0f + e)) * u;
    return __builtin_bit_cast(uint16_t, static_cast<_Float16>(y));
}

__device__ __forceinline__ float f16_bits_to_f32(uint32_t bits16) {
    return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(bits16)));
}

// A pointer into memory this kernel does not write, as a constant-address-space pointer (scalar loads)
template <class T>
__device__ __forceinline__ const __attribute__((address_space(4))) T* const_ptr(const T* p) {
    return (const __attribute__((address_space(4))) T*)(p);
}

__device__ __forceinline__ float group16_max(float m) {
#pragma unroll
    for (int o = 1; o < 16; o <<= 1) m = fmaxf(m, xor_lane(m, o));
    return m;
}
__device__ __forceinline__ int group16_sum(int v) {
#pragma unroll
    for (int o = 1; o < 16; o <<= 1) v += xor_lane(v, o);
    return v;
}
__device__ __forceinline__ int clamp127(float r) { return int(fminf(fmaxf(r, -127.0f), 127.0f)); }

// Z' = A8(Z H512 / sqrt(512)) of one fp16 row of 512 values by one wave (engine/moe_i8.cu:447-502): lane l owns
// values 8l .. 8l+7; butterfly stages h = 1, 2, 4 in registers, h = 8 .. 256 by lane shuffles (xor 1 .. 32), in
// ascending h; the group quantiser multiplies by 1/s. Out (logical order): the lane's 8 codes, and its group's
// scale and code sum (group = lane / 16). All 64 lanes must be active.
// fwht512_a8_raw: the same from the lane's 16 bytes of the row, already loaded (raw = the row's bytes 16l .. 16l+15).
__device__ __forceinline__ void fwht512_a8_raw(const uint4& raw, int lane, uint2& qw, float& sc, int& tot) {
    const uint32_t rw[4] = {raw.x, raw.y, raw.z, raw.w};
    float x[8];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        x[2 * j] = f16_bits_to_f32(rw[j] & 0xFFFFu);
        x[2 * j + 1] = f16_bits_to_f32(rw[j] >> 16);
    }
#pragma unroll
    for (int h = 1; h < 8; h <<= 1)
#pragma unroll
        for (int j = 0; j < 8; ++j)
            if (!(j & h)) {
                const float a = x[j], b = x[j + h];
                x[j] = a + b;
                x[j + h] = a - b;
            }
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        // butterfly: the lower lane of the pair keeps x + y, the upper y - x; fma(+-1, x, y) rounds exactly
        // like that sum or difference
        const float sg = (lane & o) ? -1.0f : 1.0f;
#pragma unroll
        for (int j = 0; j < 8; ++j) x[j] = __builtin_fmaf(sg, x[j], xor_lane(x[j], o));
    }
    float m = 0.0f;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        x[j] = x[j] * 0.04419417382415922f;
        m = fmaxf(m, fabsf(x[j]));
    }
    m = group16_max(m);
    sc = fmaxf(m / 127.0f, 1e-30f);
    const float inv = 1.0f / sc;
    int t = 0;
    uint32_t w0 = 0, w1 = 0;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        const int qq = clamp127(__builtin_rintf(x[j] * inv));
        t += qq;
        if (j < 4) w0 |= uint32_t(qq & 0xFF) << (8 * j);
        else w1 |= uint32_t(qq & 0xFF) << (8 * (j - 4));
    }
    qw = make_uint2(w0, w1);
    tot = group16_sum(t);
}
__device__ __forceinline__ void fwht512_a8(const uint16_t* __restrict__ zrow, int lane, uint2& qw, float& sc, int& tot) {
    fwht512_a8_raw(*reinterpret_cast<const uint4*>(zrow + 8 * lane), lane, qw, sc, tot);
}

// A8 of 512 consecutive values by one wave (engine/ops.cu:42-66): lane l owns values 8l .. 8l+7, a 128-group is
// 16 lanes; s = max(max|v| / 127, 1e-30), q = clamp(rint(v / s), +-127). Writes the lane's 8 codes and, from the
// group's first lane, its scale and code sum (s4 / sum4: the 4 groups of the 512). All 64 lanes must be active.
// A8 of 8 values per lane, 16 lanes per 128-group (lanes 16g .. 16g+15 hold group g's values in order): the
// lane's 8 codes go to q8, and lane 16g writes its group's scale and code sum to *s and *sum (nothing is written
// when store is false).
__device__ __forceinline__ void quant_a8_8(const float (&v)[8], int lane, int8_t* __restrict__ q8,
                                           float* __restrict__ s, int* __restrict__ sum, bool store = true) {
    float m = 0.0f;
#pragma unroll
    for (int j = 0; j < 8; ++j) m = fmaxf(m, fabsf(v[j]));
    m = group16_max(m);
    const float sc = fmaxf(m / 127.0f, 1e-30f);
    int tot = 0;
    uint32_t w0 = 0, w1 = 0;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        const int qq = clamp127(__builtin_rintf(v[j] / sc));
        tot += qq;
        if (j < 4) w0 |= uint32_t(qq & 0xFF) << (8 * j);
        else w1 |= uint32_t(qq & 0xFF) << (8 * (j - 4));
    }
    if (store) *reinterpret_cast<uint2*>(q8) = make_uint2(w0, w1);
    tot = group16_sum(tot);
    if (store && (lane & 15) == 0) {
        *s = sc;
        *sum = tot;
    }
}
__device__ __forceinline__ void quant_a8_512(const float* __restrict__ x, int lane, int8_t* __restrict__ q,
                                             float* __restrict__ s4, int* __restrict__ sum4) {
    const float4 a = *reinterpret_cast<const float4*>(x + 8 * lane);
    const float4 b = *reinterpret_cast<const float4*>(x + 8 * lane + 4);
    const float v[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
    quant_a8_8(v, lane, q + 8 * lane, s4 + (lane >> 4), sum4 + (lane >> 4));
}

// the A8 of the layer input (H = 2048) done by the first per-token routing kernel when routing from given logits
struct QuantX {
    const float* x;     // [T, 2048] fp32, nullptr: no A8
    int8_t* q;
    float* s;
    int* sum;
};

// ---- host launchers (each returns the launch's hipError_t) ----

struct GemmArgs {
    const uint8_t* base;        // device weight arena
    const uint64_t* off;        // [E+1] byte offset of the matrix of each expert (gate_up or down)
    const int8_t* bits;         // [E+1]
    const Item* items;          // work units
    const int* n_items;         // device count of work units (the persistent grid loops over them)
    const int* slot_token;      // gate_up: B row of slot s is token slot_token[s]; nullptr: row = slot
    const int8_t* xq;           // B rows, int8 [rows, K]
    const float* xs;            // [rows, K/128]
    const int* xsum;            // [rows, K/128]
    const float* slot_weight;   // down: Y = w_slot * acc
    int K;                      // reduction length (H for gate_up, I for down)
    int R;                      // output rows (2I for gate_up, H for down)
    uint16_t* Z;                // gate_up out [slots, R/2] fp16
    float* Y;                   // down out [slots, R]
    uint16_t* Yh;               // down, fast numerics: out as fp16 [slots, R] (round to nearest even) instead of Y
    int32_t* P;                 // group-products out [n, R, K/128] (test entry)
    const int* tstart;          // tiled: [G + 1] first task of each workgroup (the work partition above)
    int accumulate;             // GEMM_DENSE: Y += acc instead of Y = acc
    int dense_T;                // dense projection at T <= 32 (launch_dense_splitk): the tokens
    int fast;                   // gate_up: SiLU by the hardware exp / reciprocal and fp16 conversion
    // streamed down GEMM: with zin set, the B rows are staged as A8(FWHT-512(zin[slot])) instead of read from xq / xs /
    // xsum, and the units of row block 0 also write those rows to xq_out / xs_out / xsum_out
    const uint16_t* zin;
    int8_t* xq_out;
    float* xs_out;
    int* xsum_out;
    // streamed down GEMM after a self-planned gate_up: workgroup 0 zeroes clear_a / clear_b [nclear] (the decode
    // routing state that the gate_up GEMM read)
    uint32_t* clear_a;
    uint32_t* clear_b;
    int nclear;
};

// The down GEMM's slot outputs w acc of one lane (4 consecutive rows from element index i): fp32 into Y, or, with
// fast numerics, rounded to fp16 (nearest even) into Yh
// Stores that every lane issues: a lane whose `ok` is false writes nothing (its byte offset is moved past the
// buffer's 2^31 - 1 byte range, and the hardware drops an out-of-range buffer store). A store inside a divergent
// branch may or may not have been issued, so the compiler's waits for later loads must also wait for it; these do
// not. `base` must be the same for the whole wave (scalar values only), offsets below 2^31.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t store_rsrc(const void* base) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, 0x7fffffff, 0x00020000);
}
__device__ __forceinline__ uint32_t store_off(uint32_t byte_off, bool ok) {
    return byte_off + (uint32_t(!ok) << 31);
}
__device__ __forceinline__ void store_b32_if(__amdgpu_buffer_rsrc_t r, uint32_t byte_off, bool ok, uint32_t v) {
    __builtin_amdgcn_raw_buffer_store_b32(v, r, store_off(byte_off, ok), 0, 0);
}
__device__ __forceinline__ void store_slot_out(const GemmArgs& a, size_t i, float w, float a0, float a1, float a2,
                                               float a3) {
    if (a.Yh) {
        const uint32_t h0 = f32_to_f16_rne(w * a0) | (uint32_t(f32_to_f16_rne(w * a1)) << 16);
        const uint32_t h1 = f32_to_f16_rne(w * a2) | (uint32_t(f32_to_f16_rne(w * a3)) << 16);
        *reinterpret_cast<uint2*>(a.Yh + i) = make_uint2(h0, h1);
    } else {
        *reinterpret_cast<float4*>(a.Y + i) = make_float4(w * a0, w * a1, w * a2, w * a3);
    }
}

// GEMM_DENSE: a plain W.A8 projection [R, 2048] (rows in packlib order), out Y[token, r] = acc (or += acc)
enum GemmMode { GEMM_GATE_UP = 0, GEMM_DOWN = 1, GEMM_PRODUCTS_GATE_UP = 2, GEMM_PRODUCTS_DOWN = 3, GEMM_DENSE = 4 };

// records msg as the calling thread's last error (llmoe_last_error) and returns code
int set_error(int code, const char* msg);
// the GEMM kernels' function attributes, once per process (LLMOE_OK or an error recorded as above)
int ensure_gemm_setup();
// packlib "i8" bytes of an [R, K] matrix of b-bit codes (-1 tile bytes: unsupported width)
int tile_wbytes(int bits);
size_t packlib_matrix_bytes(int R, int K, int bits);

hipError_t gemm_setup();   // function attributes (dynamic LDS), once per process
hipError_t launch_expert_gemm(int mode, int nt, const GemmArgs& a, int max_items, hipStream_t st);
// dense projection at T = a.dense_T <= 32 (K = 2048), split over K (one superblock per wave)
hipError_t launch_dense_splitk(int bits, const GemmArgs& a, hipStream_t st);
// the decode gate_up GEMM that builds the slot plan itself from the routing masks (a.items / a.n_items unused), and
// writes the plan's lists (DecodePlanArgs::d) for the down GEMM and the combine
struct DecodePlanArgs;
hipError_t launch_expert_gemm_plan(const GemmArgs& a, const DecodePlanArgs& p, hipStream_t st);
// tiled units (a.items / a.n_items): mode GEMM_GATE_UP or GEMM_DOWN
hipError_t tiled_setup();
// resident workgroups of the tiled GEMM grid for mode GEMM_GATE_UP / GEMM_DOWN (the G of the work partition)
int tiled_grid(int mode);
hipError_t launch_tiled_gemm(int mode, const GemmArgs& a, hipStream_t st);
hipError_t launch_relayout(const uint8_t* src, uint8_t* dst, int R, int K, int bits, int gate_up, hipStream_t st);
hipError_t launch_quant_a8(const float* x, int rows, int cols, int8_t* q, float* s, int* sum, hipStream_t st);
// every finite fp32 input through f32_to_f16_rne and f32_to_f16_bits; differences counted into *mismatches
hipError_t launch_f16_selftest(unsigned long long* mismatches, hipStream_t st);
hipError_t launch_fwht_a8(const uint16_t* Z, int nslots, int8_t* q, float* s, int* sum, hipStream_t st);
// combine + FWHT-2048 un-rotation + residual into h + next-layer RMSNorm / rotation / A8 (H = 2048)
// (Y: fp32 [S, H], or fp16 bits when yhalf is set -- the down GEMM's fast-numerics output)
hipError_t launch_combine_norm(const void* Y, int yhalf, const int* tok_slots, int T, int kk, int K1,
                               const float* signs, float eps, float* h, int8_t* q, float* s, int* sum, hipStream_t st);
hipError_t launch_combine(const void* Y, int yhalf, const int* tok_slots, int T, int H, int kk, int K1, float* out,
                          hipStream_t st);
// router logits partials; with q != nullptr also the A8 of x (q, qs, qsum as launch_quant_a8), H = 2048
hipError_t launch_router_logits(const float* x, const float* Wr, int T, int H, int E, float* part, int8_t* q,
                                float* qs, int* qsum, hipStream_t st);
hipError_t launch_route(const float* part, int nchunks, const float* bias, int T, int E, int K, int C, int block,
                        float rscale, float* sig, uint32_t* blockmax, int32_t* topk, float* topw, uint32_t* mask,
                        const QuantX& qx, hipStream_t st);
// decode step (T <= 32, one routing block): [scores and pool keys (pool < E)], selection in ceil(T/8)
// workgroups, then (dispatch != 0) one workgroup builds the slots and work units (streamed, 16 slots per item).
// blockmax / tmask [E] must be zero on entry and are zero again on exit when dispatch is set; otherwise the gate_up
// GEMM plans from them (launch_expert_gemm_plan) and the down GEMM clears them. sig: [T, E] scratch.
hipError_t launch_decode_route(const float* part, int nchunks, const float* bias, int T, int E, int K, int C,
                               float rscale, float* sig, int32_t* topk, float* topw, uint32_t* blockmax,
                               uint32_t* tmask, int has_shared, const int8_t* bits, int32_t* count, int32_t* start,
                               Item* units_gu, Item* units_dn, int* n_units, int32_t* slot_token, float* slot_weight,
                               int32_t* tok_slots, const QuantX& qx, int dispatch, hipStream_t st);
// zero the decode routing state (blockmax, tmask [E]) when no kernel of the step consumed it
hipError_t launch_zero_decode_state(uint32_t* blockmax, uint32_t* tmask, int E, hipStream_t st);
hipError_t launch_masks(const int32_t* topk, int T, int E, int K, int block, uint32_t* mask, hipStream_t st);
// work units: streamed units_gu / units_dn (n_units[0] / [1], items of <= ntok slots); when `tiled` is set, the
// chunks of the experts with more than TILED_MIN slots in tunits_gu / tunits_dn (n_units[2] / [3], Item.rb =
// the chunk's position pre_i) and the work partition of the two tiled grids (g_gu / g_dn workgroups):
// tstart[0 .. g_gu] for gate_up, tstart[g_gu + 1 .. g_gu + 1 + g_dn] for down. max_chunks bounds the chunk count
// (dynamic LDS).
hipError_t launch_plan(const uint32_t* mask, int T, int E, int K, int block, int has_shared, int ntok, int tiled,
                       const int8_t* bits, int32_t* count, int32_t* start, int32_t* bpre, Item* units_gu,
                       Item* units_dn, Item* tunits_gu, Item* tunits_dn, int* n_units, int g_gu, int g_dn,
                       int* tstart, int max_chunks, hipStream_t st);
hipError_t launch_place(const int32_t* topk, const float* topw, uint32_t* mask, uint32_t* blockmax,
                        const int32_t* bpre, int T, int E, int K, int block, int has_shared, int32_t* slot_token,
                        float* slot_weight, int32_t* tok_slots, hipStream_t st);

}  // namespace llmoe
