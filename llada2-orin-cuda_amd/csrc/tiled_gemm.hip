// Tiled routed-expert W(2/3/4/8)·A8 GEMMs for experts with many tokens (prefill / batched denoising), gfx950
// int8 MFMA. Same math and the same fp32 operation sequence as expert_gemm.hip (engine/moe_i8.cu:1-14,
// :364-383): per 128-group g, P_g = sum code xq - zero Sxq exact in int32, then
// acc = fma(scale_w scale_x, float(P_g), acc) for g ascending from 0.
//
// Work unit: <= TILED_NTOK (64) slots of one expert and a range of row blocks. The workgroup (8 waves; 16 for
// down) first copies the chunk's int8 activation rows for the WHOLE reduction (64 x K bytes, XOR-swizzled 16-byte
// chunks so the MFMA operand reads are conflict-free), their scales and sums into LDS, then every wave streams
// its own tiled_spw 16-row strips of each row block through registers: each 16x128 weight tile is unpacked once
// into MFMA A operands and used for all 4 token tiles, and the fp32 accumulators of the (strip, token tile) pairs
// stay in registers until the fused epilogue. No barrier inside a row block, so the waves (2 per SIMD; 4 for
// down) drift freely and one wave's MFMAs overlap another's vector epilogue.
// Zero points: for 2/3-bit codes the zero is subtracted while unpacking (a v_perm_b32 lookup of c - z), for 4-bit
// codes bytewise (c + 128 - z, then ^ 0x80) when the tile serves two or more token tiles; 8-bit codes (stored
// c - 128) and 4-bit codes of one-tile chunks put the zero term zero * (-Sxq) of the lane's four output rows on the
// MFMA's initial accumulator instead. Either way the accumulator starts from I2F_BIAS, so its bits end as the
// float 1.5 * 2^23 + P_g and one subtraction gives float(P_g).
#include <type_traits>

#include "llmoe_internal.h"

namespace llmoe {

namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef unsigned int u4 __attribute__((ext_vector_type(4)));

// waves and threads per workgroup of the GEMM with reduction K
__host__ __device__ constexpr int nw_for(int K) { return tiled_waves(K == 512); }
__host__ __device__ constexpr int nthreads_for(int K) { return 64 * nw_for(K); }
constexpr int MAX_TILE = TILED_NTOK / 16;       // 16-token tiles per chunk
// LDS: activations [group][token][128 B] (16-byte chunk c of token n at ((c ^ (n & 7)) * 16)), then fp32 scales
// and negated int32 sums [group][token], then the chunk's row table [token]
constexpr int GROUP_B = TILED_NTOK * GROUP;
__host__ __device__ constexpr int lds_bytes_for(int K) {
    return (K / GROUP) * (GROUP_B + TILED_NTOK * 8) + TILED_NTOK * 4;
}
// gate_up with 8-bit codes: a row block's Z ([token][8 fp16 per strip of the row block], rows padded by 16 bytes so
// that the 16 token columns of a store fall in different banks) goes through LDS and is stored as whole row segments
__host__ __device__ constexpr int zbuf_pitch(int spw) { return 4 * tiled_waves(false) * spw + 4; }   // uint32
constexpr int ZBUF_BYTES = TILED_NTOK * zbuf_pitch(1) * 4;
__host__ __device__ constexpr int mode_lds_bytes(int mode) {
    return mode == GEMM_DOWN ? lds_bytes_for(512) : lds_bytes_for(2048) + (mode == GEMM_GATE_UP ? ZBUF_BYTES : 0);
}
constexpr int NXCD = 8;   // XCDs of MI355X (accelerator complex dies, each with its own L2)

template <int I, int N, class F>
__device__ __forceinline__ void static_for(F&& f) {
    if constexpr (I < N) {
        f(std::integral_constant<int, I>{});
        static_for<I + 1, N>(f);
    }
}

// The weight data of one strip-superblock held by one lane, split by when it can be refilled with the next
// superblock: codes (BITS dwordx4; the 3-bit high plane lives in Late) and the fp16 scales of tiles 0-1 are
// refilled group by group as soon as a tile has been unpacked; the scales of tiles 2-3, the zeros and the 3-bit
// high plane serve all four tiles and are double-buffered a superblock ahead.
template <int BITS>
struct Codes {
    static constexpr int N = BITS == 3 ? 2 : BITS;
    u4 c[N];
    u4 s0;          // fp16 scales [tile 0-1][rows 4q .. 4q+3]
};
struct Late {
    u4 s1;          // fp16 scales [tile 2-3][rows 4q .. 4q+3]
    u4 z;           // zeros: 2/3-bit the lane's A-operand row (byte r%4 of dword tile), 4/8-bit its 4 output rows
    u4 hi;          // 3-bit high plane
};

template <int BITS>
__device__ __forceinline__ void load_code(const uint8_t* p, int lane, int i, Codes<BITS>& r) {
    r.c[i] = __builtin_nontemporal_load(reinterpret_cast<const u4*>(p + i * 1024) + lane);
}
template <int BITS>
__device__ __forceinline__ void load_s0(const uint8_t* p, int lane, Codes<BITS>& r) {
    r.s0 = *reinterpret_cast<const u4*>(p + BITS * 1024 + 32 * (lane >> 4));
}
// ZACC: the zero term rides on the MFMA accumulator (zeros of the lane's four output rows); otherwise the zero is
// subtracted while unpacking (zeros of the lane's A-operand row)
template <int BITS, bool ZACC>
__device__ __forceinline__ void load_late(const uint8_t* p, int lane, Late& r) {
    const uint8_t* m = p + BITS * 1024;
    r.s1 = *reinterpret_cast<const u4*>(m + 32 * (lane >> 4) + 16);
    r.z = *reinterpret_cast<const u4*>(m + 128 + 16 * (ZACC ? (lane >> 4) : ((lane & 15) >> 2)));
    if constexpr (BITS == 3) r.hi = __builtin_nontemporal_load(reinterpret_cast<const u4*>(p + 2 * 1024) + lane);
}

// A operand dwords of tile tau (D[0..3]: columns 0..63, D[4..7]: 64..127). 2/3-bit: the codes select bytes of a
// table holding c - z for every code c (v_perm_b32). The 2-bit table is the 4-byte window at offset 3 - z of
// the byte sequence -3 .. 3 (one v_alignbyte_b32); the 3-bit table is built as (c | 0x80) - z per byte, which
// never borrows across bytes (c + 128 - z > 0), with ^ 0x80 turning the biased byte into the two's complement
// of c - z. 4/8-bit: the codes as they are (the zero term is on the accumulator).
template <int BITS, bool ZACC>
__device__ __forceinline__ void unpack_a(const Codes<BITS>& r, const Late& lt, int tau, int lane, uint32_t (&D)[8]) {
    if constexpr (BITS == 8) {
        const u4& a = r.c[2 * tau];
        const u4& b = r.c[2 * tau + 1];
        D[0] = a.x; D[1] = a.y; D[2] = a.z; D[3] = a.w;
        D[4] = b.x; D[5] = b.y; D[6] = b.z; D[7] = b.w;
    } else {
        if constexpr (BITS == 2 || BITS == 3) {
            // codes 0 .. 2^BITS - 1 select bytes of a table holding c - z for every code (v_perm_b32)
            const u4& u = r.c[tau >> 1];
            const uint32_t p0 = (tau & 1) ? u.z : u.x, p1 = (tau & 1) ? u.w : u.y;
#pragma unroll
            for (int s = 0; s < 4; ++s) {
                D[s] = (p0 >> (2 * s)) & 0x03030303u;
                D[4 + s] = (p1 >> (2 * s)) & 0x03030303u;
            }
            if constexpr (BITS == 3) {
                const uint32_t h = lt.hi[tau];
#pragma unroll
                for (int s = 0; s < 8; ++s) {
                    const uint32_t hb = s >= 2 ? (h >> (s - 2)) : (h << (2 - s));
                    D[s] |= hb & 0x04040404u;
                }
            }
            if constexpr (BITS == 2) {
                // alignbyte reads only bits 1:0 of the shift: (z ^ 3) = 3 - z for z in 0 .. 3
                const uint32_t sh = (lt.z[tau] >> (8 * (lane & 3))) ^ 3u;
                const uint32_t t = __builtin_amdgcn_alignbyte(0x00030201u, 0x00FFFEFDu, sh);   // c - z, c = 0 .. 3
#pragma unroll
                for (int s = 0; s < 8; ++s) D[s] = __builtin_amdgcn_perm(0u, t, D[s]);
            } else {
                const uint32_t z = (lt.z[tau] >> (8 * (lane & 3))) & 0xFFu;
                const uint32_t zb = z * 0x01010101u;
                const uint32_t t_lo = ((0x03020100u | 0x80808080u) - zb) ^ 0x80808080u;   // c - z, c = 0 .. 3
                const uint32_t t_hi = ((0x07060504u | 0x80808080u) - zb) ^ 0x80808080u;   // c = 4 .. 7
#pragma unroll
                for (int s = 0; s < 8; ++s) D[s] = __builtin_amdgcn_perm(t_hi, t_lo, D[s]);
            }
            return;
        } else if constexpr (ZACC) {
            const u4& u = r.c[tau];
#pragma unroll
            for (int m = 0; m < 4; ++m) {
                D[2 * m] = u[m] & 0x0F0F0F0Fu;
                D[2 * m + 1] = (u[m] >> 4) & 0x0F0F0F0Fu;
            }
        } else {
            // c + 128 - z per byte never borrows across bytes (c, z in 0 .. 15); ^ 0x80 gives the int8 c - z
            const u4& u = r.c[tau];
            const uint32_t z = (lt.z[tau] >> (8 * (lane & 3))) & 0xFFu;
            const uint32_t k = 0x80808080u - z * 0x01010101u;
#pragma unroll
            for (int m = 0; m < 4; ++m) {
                D[2 * m] = ((u[m] & 0x0F0F0F0Fu) + k) ^ 0x80808080u;
                D[2 * m + 1] = (((u[m] >> 4) & 0x0F0F0F0Fu) + k) ^ 0x80808080u;
            }
        }
    }
}

// refill, after tile tau of a superblock has been unpacked, the code / scale registers only tile tau used with
// the next superblock at p
template <int BITS, int TAU>
__device__ __forceinline__ void refill_after(const uint8_t* p, int lane, Codes<BITS>& r) {
    if constexpr (BITS == 8) {
        load_code<BITS>(p, lane, 2 * TAU, r);
        load_code<BITS>(p, lane, 2 * TAU + 1, r);
    } else if constexpr (BITS == 4) {
        load_code<BITS>(p, lane, TAU, r);
    } else if constexpr (TAU & 1) {
        load_code<BITS>(p, lane, TAU >> 1, r);
    }
    if constexpr (TAU == 1) load_s0<BITS>(p, lane, r);
}

__device__ __forceinline__ float mul_f16_f32(uint32_t packed, int hi, float x) {
    float r;
    if (hi) asm("v_fma_mix_f32 %0, %1, %2, %3 op_sel:[1,0,0] op_sel_hi:[1,0,0]" : "=v"(r) : "v"(packed), "v"(x), "v"(-0.0f));
    else asm("v_fma_mix_f32 %0, %1, %2, %3 op_sel_hi:[1,0,0]" : "=v"(r) : "v"(packed), "v"(x), "v"(-0.0f));
    return r;
}

// The chunk's activations for the whole reduction -> LDS (all threads; rows of absent tokens are zero, so their
// MFMA columns are zero). The chunk's row indices go through a small LDS table first, so that every thread then
// issues all of its activation loads back to back. Returns after the workgroup barrier.
template <int K>
__device__ __forceinline__ void stage_chunk(const GemmArgs& a, const Item& it, uint8_t* lds) {
    constexpr int NTHREADS = nthreads_for(K);
    constexpr int G = K / GROUP, PER = TILED_NTOK * (K / 16) / NTHREADS;
    constexpr int PS = (G * TILED_NTOK + NTHREADS - 1) / NTHREADS;
    static_assert(PER * NTHREADS == TILED_NTOK * (K / 16) && TILED_NTOK == 64, "staging split");
    // the staging addresses are recomputed per chunk (a few VALU): hoisted out of the chunk loop they would stay
    // live across every row block and be spilled
    int tid = threadIdx.x;
    asm volatile("" : "+v"(tid));
    float* ss = reinterpret_cast<float*>(lds + G * GROUP_B);
    int* sq = reinterpret_cast<int*>(ss + G * TILED_NTOK);
    int* rowtab = sq + G * TILED_NTOK;
    if (tid < TILED_NTOK)
        rowtab[tid] = tid < it.ntok ? (a.slot_token ? a.slot_token[it.slot0 + tid] : it.slot0 + tid) : -1;
    __syncthreads();
    // thread chunk idx: a wave's 64 lanes cover 8 tokens x the 8 16-byte chunks of one group, i.e. one
    // contiguous, bank-conflict-free KiB of LDS; consecutive lanes read 128 contiguous bytes of a row
    auto chunk = [&](int idx, int& n, int& g, int& c16) {
        const int b = idx >> 6, l = idx & 63;
        g = b >> 3;
        n = ((b & 7) << 3) + (l >> 3);
        c16 = l & 7;
    };
    u4 v[PER];
#pragma unroll
    for (int i = 0; i < PER; ++i) {
        int n, g, c16;
        chunk(tid + NTHREADS * i, n, g, c16);
        const int row = rowtab[n];
        v[i] = row >= 0 ? *reinterpret_cast<const u4*>(a.xq + size_t(row) * K + g * GROUP + 16 * c16)
                        : u4{0u, 0u, 0u, 0u};
    }
    float sv[PS];
    int qv[PS];
#pragma unroll
    for (int i = 0; i < PS; ++i) {
        const int idx = tid + NTHREADS * i, n = idx / G, g = idx % G;
        const int row = idx < G * TILED_NTOK ? rowtab[n] : -1;
        sv[i] = row >= 0 ? a.xs[size_t(row) * G + g] : 0.0f;
        qv[i] = row >= 0 ? -a.xsum[size_t(row) * G + g] : 0;
    }
#pragma unroll
    for (int i = 0; i < PER; ++i) {
        int n, g, c16;
        chunk(tid + NTHREADS * i, n, g, c16);
        *reinterpret_cast<u4*>(lds + g * GROUP_B + n * GROUP + ((c16 ^ (n & 7)) << 4)) = v[i];
    }
#pragma unroll
    for (int i = 0; i < PS; ++i) {
        const int idx = tid + NTHREADS * i, n = idx / G, g = idx % G;
        if (idx < G * TILED_NTOK) {
            ss[g * TILED_NTOK + n] = sv[i];
            sq[g * TILED_NTOK + n] = qv[i];
        }
    }
    __syncthreads();
}

// 4-bit codes subtract the zero while unpacking once the unpacked tile serves two or more token tiles (16 VALU per
// tile against 8 per token tile for the accumulator's zero term)
template <int BITS, int NTILE>
__host__ __device__ constexpr bool zacc() { return BITS == 8 || (BITS == 4 && NTILE == 1); }

// The weight registers of one row block (wave w's strips (rb * NW + w) * S .. + S - 1): the first superblock's
// codes and meta, and the second superblock's meta for K = 2048
template <int BITS, int MODE>
struct RowRegs {
    static constexpr int S = tiled_spw(MODE == GEMM_DOWN, BITS);
    Codes<BITS> cd[S];
    Late lt[2][S];
};

template <int BITS, int MODE, int NTILE>
__device__ __forceinline__ void rowblock_load(const uint8_t* mat, int rb, RowRegs<BITS, MODE>& r) {
    constexpr int NSB = MODE == GEMM_DOWN ? 1 : 4, S = RowRegs<BITS, MODE>::S, NW = nw_for(NSB * SB_K);
    constexpr size_t SBB = sb_bytes(BITS);
    constexpr bool ZACC = zacc<BITS, NTILE>();
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint8_t* p0 = mat + size_t((rb * NW + wave) * S) * NSB * SBB;
#pragma unroll
    for (int s = 0; s < S; ++s) {
        const uint8_t* p = p0 + size_t(s) * NSB * SBB;
#pragma unroll
        for (int i = 0; i < Codes<BITS>::N; ++i) load_code<BITS>(p, lane, i, r.cd[s]);
        load_s0<BITS>(p, lane, r.cd[s]);
        load_late<BITS, ZACC>(p, lane, r.lt[0][s]);
        if constexpr (NSB > 1) load_late<BITS, ZACC>(p + SBB, lane, r.lt[1][s]);
    }
}

// One row block's products for the chunk staged in LDS, from the registers rowblock_load filled (the later
// superblocks of K = 2048 are requested along the way): the fp32 accumulators of the wave's (strip, token tile)
// pairs.
template <int BITS, int MODE, int NTILE>
__device__ __forceinline__ void rowblock_compute(const uint8_t* mat, const uint8_t* lds, int rb,
                                                 RowRegs<BITS, MODE>& r,
                                                 float (&acc)[RowRegs<BITS, MODE>::S][NTILE][4]) {
    constexpr bool DOWN = MODE == GEMM_DOWN;
    constexpr int NSB = DOWN ? 1 : 4, K = NSB * SB_K, G = K / GROUP;
    constexpr int S = RowRegs<BITS, MODE>::S, NW = nw_for(K);
    constexpr size_t SBB = sb_bytes(BITS);
    constexpr bool ZACC = zacc<BITS, NTILE>();
    const int lane = threadIdx.x & 63, q = lane >> 4, col = lane & 15;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int strip0 = (rb * NW + wave) * S;
    auto sbp = [&](int s, int sb) { return mat + (size_t(strip0 + s) * NSB + sb) * SBB; };
    const float* ss = reinterpret_cast<const float*>(lds + G * GROUP_B);
    const int* sq = reinterpret_cast<const int*>(ss + G * TILED_NTOK);
    Codes<BITS> (&cd)[S] = r.cd;
    Late (&lt)[2][S] = r.lt;
#pragma unroll
    for (int s = 0; s < S; ++s)
#pragma unroll
        for (int nt = 0; nt < NTILE; ++nt)
#pragma unroll
            for (int v = 0; v < 4; ++v) acc[s][nt][v] = 0.0f;

    static_for<0, G>([&](auto gc) {
        constexpr int g = decltype(gc)::value, sb = g / 4, tau = g % 4;
        const uint8_t* bg = lds + g * GROUP_B;
        v4i A0[S], A1[S];
        uint32_t swp[S][2];
        int zz[S][4];
#pragma unroll
        for (int s = 0; s < S; ++s) {
            const Late& l = lt[sb % 2][s];
            uint32_t Dw[8];
            unpack_a<BITS, ZACC>(cd[s], l, tau, lane, Dw);
            A0[s] = v4i{int(Dw[0]), int(Dw[1]), int(Dw[2]), int(Dw[3])};
            A1[s] = v4i{int(Dw[4]), int(Dw[5]), int(Dw[6]), int(Dw[7])};
            const u4& sv = tau < 2 ? cd[s].s0 : l.s1;
            swp[s][0] = sv[(tau & 1) * 2];
            swp[s][1] = sv[(tau & 1) * 2 + 1];
            if constexpr (ZACC) {
#pragma unroll
                for (int v = 0; v < 4; ++v) zz[s][v] = int((l.z[tau] >> (8 * v)) & 0xFFu) - (BITS == 8 ? 128 : 0);
            }
            // registers tile tau alone used: refill with the next superblock; after the last tile the
            // superblock-wide registers take the superblock after next
            if constexpr (sb + 1 < NSB) refill_after<BITS, tau>(sbp(s, sb + 1), lane, cd[s]);
            if constexpr (tau == 3 && sb + 2 < NSB) load_late<BITS, ZACC>(sbp(s, sb + 2), lane, lt[sb % 2][s]);
        }
        // software pipeline over the token tiles: the MFMAs of tile nt are issued before the fp32 epilogue of
        // tile nt-1, and the B operands are read one tile ahead
        auto bptr = [&](int nt, int half) {
            const int n = nt * 16 + col;
            return reinterpret_cast<const v4i*>(bg + n * GROUP + (((q + 4 * half) ^ (n & 7)) << 4));
        };
        // with several token tiles the group's fp16 weight scales are converted once and multiplied per tile
        float swf[S][4];
        if constexpr (NTILE > 1) {
#pragma unroll
            for (int s = 0; s < S; ++s)
#pragma unroll
                for (int v = 0; v < 4; ++v) swf[s][v] = f16_bits_to_f32(swp[s][v >> 1] >> (16 * (v & 1)));
        }
        v4i Cp[S];
        float xsp = 0.0f;
        v4i Bn0 = *bptr(0, 0), Bn1 = *bptr(0, 1);
        float xsnext = ss[g * TILED_NTOK + col];
        int nsnext = 0;
        if constexpr (ZACC) nsnext = sq[g * TILED_NTOK + col];
        static_for<0, NTILE + 1>([&](auto tc) {
            constexpr int nt = decltype(tc)::value;
            v4i Cc[S];
            float xsn = 0.0f;
            if constexpr (nt < NTILE) {
                const v4i B0 = Bn0, B1 = Bn1;
                xsn = xsnext;
                const int nsum = nsnext;
                if constexpr (nt + 1 < NTILE) {
                    Bn0 = *bptr(nt + 1, 0);
                    Bn1 = *bptr(nt + 1, 1);
                    xsnext = ss[g * TILED_NTOK + (nt + 1) * 16 + col];
                    if constexpr (ZACC) nsnext = sq[g * TILED_NTOK + (nt + 1) * 16 + col];
                }
#pragma unroll
                for (int s = 0; s < S; ++s) {
                    if constexpr (ZACC)
                        Cc[s] = v4i{__mul24(zz[s][0], nsum) + I2F_BIAS, __mul24(zz[s][1], nsum) + I2F_BIAS,
                                    __mul24(zz[s][2], nsum) + I2F_BIAS, __mul24(zz[s][3], nsum) + I2F_BIAS};
                    else
                        Cc[s] = v4i{I2F_BIAS, I2F_BIAS, I2F_BIAS, I2F_BIAS};
                    Cc[s] = __builtin_amdgcn_mfma_i32_16x16x64_i8(A0[s], B0, Cc[s], 0, 0, 0);
                }
#pragma unroll
                for (int s = 0; s < S; ++s) Cc[s] = __builtin_amdgcn_mfma_i32_16x16x64_i8(A1[s], B1, Cc[s], 0, 0, 0);
            }
            if constexpr (nt > 0) {
#pragma unroll
                for (int s = 0; s < S; ++s) {
#pragma unroll
                    for (int v = 0; v < 4; ++v) {
                        // scale_w * scale_x: one fp32 product either way (the fp16 scale converts exactly)
                        const float sc = NTILE > 1 ? swf[s][v] * xsp : mul_f16_f32(swp[s][v >> 1], v & 1, xsp);
                        acc[s][nt - 1][v] = __builtin_fmaf(sc, biased_to_f32(Cp[s][v]), acc[s][nt - 1][v]);
                    }
                    // materialise the tile's accumulators here: otherwise the compiler defers the fp32 chains
                    // and keeps every tile's MFMA results live
                    asm volatile("" : "+v"(acc[s][nt - 1][0]), "+v"(acc[s][nt - 1][1]), "+v"(acc[s][nt - 1][2]),
                                 "+v"(acc[s][nt - 1][3]));
                }
            }
            if constexpr (nt < NTILE) {
#pragma unroll
                for (int s = 0; s < S; ++s) Cp[s] = Cc[s];
                xsp = xsn;
            }
            __builtin_amdgcn_sched_barrier(0);
        });
    });

}

// The row block's fused epilogue: Z = fp16(SiLU(g) u) (gate_up), Y = w acc (down) or Y (+)= acc (dense). The Z
// stores are issued by every lane (absent tokens' stores dropped), so that the waits for the next row block's weights
// need not wait for them: the loop head then waits with vmcnt(10) instead of vmcnt(2) (2-bit, 4 token tiles; config 3
// gate_up -1 %).
template <int BITS, int MODE, int NTILE>
__device__ __forceinline__ void rowblock_store(const GemmArgs& a, const Item& it, int rb,
                                               const float (&acc)[RowRegs<BITS, MODE>::S][NTILE][4], uint8_t* lds) {
    constexpr int S = RowRegs<BITS, MODE>::S, NW = nw_for(MODE == GEMM_DOWN ? SB_K : 4 * SB_K);
    const int lane = threadIdx.x & 63, q = lane >> 4, col = lane & 15;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int strip0 = (rb * NW + wave) * S;
    // the chunk's rows of Z (slot0 is the same for the whole workgroup)
    const __amdgpu_buffer_rsrc_t rz =
        store_rsrc(MODE == GEMM_GATE_UP ? static_cast<const void*>(a.Z + size_t(it.slot0) * (a.R / 2)) : nullptr);
#pragma unroll
    for (int s = 0; s < S; ++s) {
        const int strip = strip0 + s;
#pragma unroll
        for (int nt = 0; nt < NTILE; ++nt) {
            const int n = nt * 16 + col;
            const bool ok = n < it.ntok;
            if constexpr (MODE == GEMM_DENSE) {
                if (ok) {
                    float4* yp = reinterpret_cast<float4*>(a.Y + size_t(it.slot0 + n) * a.R + 16 * strip + 4 * q);
                    float4 y = make_float4(acc[s][nt][0], acc[s][nt][1], acc[s][nt][2], acc[s][nt][3]);
                    if (a.accumulate) {
                        const float4 o = *yp;
                        y = make_float4(o.x + y.x, o.y + y.y, o.z + y.z, o.w + y.w);
                    }
                    *yp = y;
                }
            } else if constexpr (MODE == GEMM_GATE_UP) {
                uint32_t z0, z1;
                if (a.fast) {
                    z0 = silu_mul_f16_fast(acc[s][nt][0], acc[s][nt][1]);
                    z1 = silu_mul_f16_fast(acc[s][nt][2], acc[s][nt][3]);
                } else {
                    z0 = f32_to_f16_rne(silu_f32(acc[s][nt][0]) * acc[s][nt][1]);
                    z1 = f32_to_f16_rne(silu_f32(acc[s][nt][2]) * acc[s][nt][3]);
                }
                if constexpr (S == 1) {
                    if (ok)
                        reinterpret_cast<uint32_t*>(lds + lds_bytes_for(2048))[n * zbuf_pitch(S) + 4 * wave + q] =
                            z0 | (z1 << 16);
                } else {
                    store_b32_if(rz, uint32_t(n * (a.R / 2) + 8 * strip + 2 * q) * 2u, ok, z0 | (z1 << 16));
                }
            } else {
                // (unconditional stores here need 24 bytes of spills at the down kernel's 128 VGPRs)
                if (ok)
                    store_slot_out(a, size_t(it.slot0 + n) * a.R + 16 * strip + 4 * q, a.slot_weight[it.slot0 + n],
                                   acc[s][nt][0], acc[s][nt][1], acc[s][nt][2], acc[s][nt][3]);
            }
        }
    }
}

template <int BITS, int MODE, int NTILE>
__device__ __forceinline__ void tiled_body(const GemmArgs& a, const Item& it, const uint8_t* mat, uint8_t* lds,
                                           int rb0, int rb1) {
    constexpr int K = MODE == GEMM_DOWN ? 512 : 2048;
    // row block rb + 1's first weights are requested between rb's products and rb's stores: the weight loads then
    // precede the output stores in the in-order memory counter, so waiting for them never waits for the stores
    RowRegs<BITS, MODE> r;
    rowblock_load<BITS, MODE, NTILE>(mat, rb0, r);
    stage_chunk<K>(a, it, lds);
    for (int rb = rb0; rb < rb1; ++rb) {
        float acc[RowRegs<BITS, MODE>::S][NTILE][4];
        rowblock_compute<BITS, MODE, NTILE>(mat, lds, rb, r, acc);
        // (8-bit codes of the 16-wave down GEMM: the accumulators and a whole superblock of codes do not fit the
        // registers together, so the stores go first)
        constexpr bool LOAD_FIRST = !(MODE == GEMM_DOWN && BITS == 8);
        if (LOAD_FIRST && rb + 1 < rb1) rowblock_load<BITS, MODE, NTILE>(mat, rb + 1, r);
        // 8-bit codes (one strip per wave): the row block's Z goes through LDS and is stored as whole row segments
        // (config-4 8-bit gate_up 0.264 -> 0.250 ms; for two strips per wave the two barriers cost what it saves)
        constexpr bool ZSTAGE = MODE == GEMM_GATE_UP && RowRegs<BITS, MODE>::S == 1;
        if constexpr (ZSTAGE) __syncthreads();   // the previous row block's Z has been read
        rowblock_store<BITS, MODE, NTILE>(a, it, rb, acc, lds);
        if constexpr (ZSTAGE) {
            __syncthreads();
            // each token's 8 NW Z values of the row block are contiguous in Z: 16 bytes (one strip) per thread
            constexpr int S = RowRegs<BITS, MODE>::S, NCH = S * tiled_waves(false);
            const uint32_t* zb = reinterpret_cast<const uint32_t*>(lds + lds_bytes_for(2048));
            for (int idx = threadIdx.x; idx < it.ntok * NCH; idx += nthreads_for(K)) {
                const int n = idx / NCH, c = idx % NCH;
                *reinterpret_cast<uint4*>(a.Z + size_t(it.slot0 + n) * (a.R / 2) + 8 * (rb * NCH + c)) =
                    *reinterpret_cast<const uint4*>(zb + n * zbuf_pitch(S) + 4 * c);
            }
        }
        if (!LOAD_FIRST && rb + 1 < rb1) rowblock_load<BITS, MODE, NTILE>(mat, rb + 1, r);
    }
}

// Workgroup w runs the row-block tasks tstart[w] .. tstart[w + 1] (chunk-major, so the chunk's activations are
// staged once per run of its row blocks).
template <int MODE>
__global__ void __launch_bounds__(nthreads_for(MODE == GEMM_DOWN ? 512 : 2048)) tiled_gemm(GemmArgs a) {
    extern __shared__ __align__(16) uint8_t lds[];
    constexpr int CMASK = (1 << TASK_RB_SHIFT) - 1;
    // XCD-aware: workgroups are dispatched round-robin over the 8 XCDs, so partition p runs on workgroup
    // (p % per) * 8 + p / per: each XCD takes a contiguous run of the (chunk-major) task list, and the chunks of a
    // hot expert -- listed one after another -- share that XCD's L2 for the expert's weights
    const int G = gridDim.x;
    const int p = G % NXCD ? int(blockIdx.x) : int(blockIdx.x % NXCD) * (G / NXCD) + int(blockIdx.x / NXCD);
    const int s0 = *const_ptr(a.tstart + p), s1 = *const_ptr(a.tstart + p + 1);
    const int c0 = s0 & CMASK, r0 = s0 >> TASK_RB_SHIFT, c1 = s1 & CMASK, r1 = s1 >> TASK_RB_SHIFT;
    for (int c = c0; c < c1 || (c == c1 && r1 > 0); ++c) {
        // the chunk, and the expert's matrix offset and code width together, by scalar loads (the lists are
        // written by earlier kernels only)
        const auto* ip = const_ptr(reinterpret_cast<const int*>(a.items + c));
        const Item it{ip[0], ip[1], ip[2], ip[3]};
        const uint64_t off = *const_ptr(a.off + it.expert);
        const uint32_t bw4 = *const_ptr(reinterpret_cast<const uint32_t*>(a.bits) + (it.expert >> 2));
        asm volatile("" ::"s"(off), "s"(bw4));
        const int bits = int(bw4 >> (8 * (it.expert & 3))) << 24 >> 24;
        const uint8_t* mat = a.base + off;
        const int nrb = MODE == GEMM_DENSE ? a.R / (16 * tiled_waves(false) * tiled_spw(false, bits))
                                           : tiled_row_blocks(MODE == GEMM_DOWN, bits);
        const int rb0 = c == c0 ? r0 : 0, rb1 = c == c1 ? r1 : nrb;
        if (rb0 >= rb1) continue;
        // token tiles actually present (a chunk has <= 64 slots; absent tiles are not computed)
        const int nt = (it.ntok + 15) >> 4;
        if (nt > 3) {
            if (bits == 2) tiled_body<2, MODE, 4>(a, it, mat, lds, rb0, rb1);
            else if (bits == 3) tiled_body<3, MODE, 4>(a, it, mat, lds, rb0, rb1);
            else if (bits == 4) tiled_body<4, MODE, 4>(a, it, mat, lds, rb0, rb1);
            else tiled_body<8, MODE, 4>(a, it, mat, lds, rb0, rb1);
        } else if (nt == 3) {
            if (bits == 2) tiled_body<2, MODE, 3>(a, it, mat, lds, rb0, rb1);
            else if (bits == 3) tiled_body<3, MODE, 3>(a, it, mat, lds, rb0, rb1);
            else if (bits == 4) tiled_body<4, MODE, 3>(a, it, mat, lds, rb0, rb1);
            else tiled_body<8, MODE, 3>(a, it, mat, lds, rb0, rb1);
        } else if (nt == 2) {
            if (bits == 2) tiled_body<2, MODE, 2>(a, it, mat, lds, rb0, rb1);
            else if (bits == 3) tiled_body<3, MODE, 2>(a, it, mat, lds, rb0, rb1);
            else if (bits == 4) tiled_body<4, MODE, 2>(a, it, mat, lds, rb0, rb1);
            else tiled_body<8, MODE, 2>(a, it, mat, lds, rb0, rb1);
        } else {
            if (bits == 2) tiled_body<2, MODE, 1>(a, it, mat, lds, rb0, rb1);
            else if (bits == 3) tiled_body<3, MODE, 1>(a, it, mat, lds, rb0, rb1);
            else if (bits == 4) tiled_body<4, MODE, 1>(a, it, mat, lds, rb0, rb1);
            else tiled_body<8, MODE, 1>(a, it, mat, lds, rb0, rb1);
        }
        __syncthreads();   // the next chunk re-stages the activations
    }
}

template <int MODE>
const void* kptr() { return reinterpret_cast<const void*>(&tiled_gemm<MODE>); }

template <int MODE>
int grid_t() {
    static int grid = 0;
    if (!grid) {
        int dev = 0, cus = 0, per_cu = 0;
        hipError_t e = hipGetDevice(&dev);
        if (e == hipSuccess) e = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
        if (e == hipSuccess)
            e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kptr<MODE>(), nthreads_for(MODE == GEMM_DOWN ? 512 : 2048),
                                                             mode_lds_bytes(MODE));
        if (e != hipSuccess) return 0;
        grid = cus * (per_cu > 0 ? per_cu : 1);
    }
    return grid;
}

template <int MODE>
hipError_t launch_t(const GemmArgs& a, hipStream_t st) {
    const int grid = grid_t<MODE>();
    if (!grid) return hipErrorInvalidDevice;
    constexpr int K = MODE == GEMM_DOWN ? 512 : 2048;
    tiled_gemm<MODE><<<grid, nthreads_for(K), mode_lds_bytes(MODE), st>>>(a);
    return hipGetLastError();
}

}  // namespace

hipError_t tiled_setup() {
    hipError_t e = hipFuncSetAttribute(kptr<GEMM_GATE_UP>(), hipFuncAttributeMaxDynamicSharedMemorySize,
                                       mode_lds_bytes(GEMM_GATE_UP));
    if (e == hipSuccess)
        e = hipFuncSetAttribute(kptr<GEMM_DOWN>(), hipFuncAttributeMaxDynamicSharedMemorySize, mode_lds_bytes(GEMM_DOWN));
    if (e == hipSuccess)
        e = hipFuncSetAttribute(kptr<GEMM_DENSE>(), hipFuncAttributeMaxDynamicSharedMemorySize, mode_lds_bytes(GEMM_DENSE));
    return e;
}

int tiled_grid(int mode) {
    return mode == GEMM_DOWN ? grid_t<GEMM_DOWN>() : mode == GEMM_DENSE ? grid_t<GEMM_DENSE>() : grid_t<GEMM_GATE_UP>();
}

hipError_t launch_tiled_gemm(int mode, const GemmArgs& a, hipStream_t st) {
    if (mode == GEMM_GATE_UP) return launch_t<GEMM_GATE_UP>(a, st);
    if (mode == GEMM_DOWN) return launch_t<GEMM_DOWN>(a, st);
    if (mode == GEMM_DENSE) return launch_t<GEMM_DENSE>(a, st);
    return hipErrorInvalidValue;
}

}  // namespace llmoe
