// Routed-expert W(2/3/4/8)·A8 GEMMs on gfx950 int8 MFMA (v_mfma_i32_16x16x64_i8).
//
// Math (engine/moe_i8.cu:1-14, :364-383): per 128-group g of the reduction
//     P_g[r, n] = sum_{k in g} code[r, k] xq[n, k] - zero[r, g] Sxq[n, g]          (exact int32)
//     acc[r, n] = fma(scale_w[r, g] * scale_x[n, g], float(P_g[r, n]), acc[r, n])  (fp32, g ascending from 0)
// The zero-point term enters as the MFMA's initial accumulator, so no integer work follows the MFMA.
// 8-bit codes are stored as code - 128 (signed), and their zero as zero - 128 in the same product.
//
// Work decomposition (one work item = up to 16*NT slots of ONE expert, so the expert's weights stream from HBM
// once per item): grid (row blocks, items); a workgroup = 4 waves; wave w owns SPW 16-row strips of the row block
// (w, w + 4, ...) and streams them through a register ring (dwordx4 loads, 1 KiB contiguous per wave and load). The item's B rows
// (int8 activations + per-group scales and sums) are staged once per workgroup in LDS. Each superblock's scales
// and zeros travel with its codes through the ring (one dword per lane) and reach the lanes through a 192-byte LDS
// slot of the wave, so the LDS holds no per-strip meta (36 KiB per workgroup at 16 tokens and K = 2048).
//   gate_up (MODE 0): rows 2I = 1024, K = H = 2048; out Z[slot, i] = fp16(SiLU(g_i) u_i)
//                     (engine/moe_i8.cu:219-221)
//   down    (MODE 1): rows H = 2048, K = I = 512; out Y[slot, h] = w_slot acc (engine/moe_i8.cu:222-231)
//   products (MODE 2, 3): raw P_g per (token, row, group) in either geometry, for the bit-exactness test.
#include <type_traits>

#include "decode_plan.h"

namespace llmoe {

namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef unsigned int u4 __attribute__((ext_vector_type(4)));

constexpr int WAVES = GEMM_WAVES;

template <int I, int N, class F>
__device__ __forceinline__ void static_for(F&& f) {
    if constexpr (I < N) {
        f(std::integral_constant<int, I>{});
        static_for<I + 1, N>(f);
    }
}

template <int BITS>
struct Step {               // one strip-superblock as held by one lane: code bytes, and dword `lane` of its meta
    u4 c[BITS];
    uint32_t m;             // lanes 0 .. 47: the 192 meta bytes (scales, zeros), passed on through the wave's LDS slot
};

template <int BITS>
__device__ __forceinline__ void load_step(const uint8_t* sbp, int lane, Step<BITS>& r) {
#pragma unroll
    for (int i = 0; i < BITS; ++i) r.c[i] = __builtin_nontemporal_load(reinterpret_cast<const u4*>(sbp + i * 1024) + lane);
    if (lane < META_SB / 4) r.m = __builtin_nontemporal_load(reinterpret_cast<const uint32_t*>(sbp + BITS * 1024) + lane);
}

__device__ __forceinline__ uint32_t wsel(const u4& v, int i) { return v[i]; }

// The 8 A-operand dwords of tile tau: D[0..3] feed the MFMA of columns 0..63, D[4..7] columns 64..127.
template <int BITS>
__device__ __forceinline__ void unpack_tile(const Step<BITS>& r, int tau, uint32_t (&D)[8]) {
    if constexpr (BITS == 2 || BITS == 3) {
        const u4& u = r.c[tau >> 1];
        const uint32_t p0 = (tau & 1) ? u.z : u.x, p1 = (tau & 1) ? u.w : u.y;
#pragma unroll
        for (int s = 0; s < 4; ++s) {
            D[s] = (p0 >> (2 * s)) & 0x03030303u;
            D[4 + s] = (p1 >> (2 * s)) & 0x03030303u;
        }
        if constexpr (BITS == 3) {
            const uint32_t h = wsel(r.c[2], tau);
#pragma unroll
            for (int s = 0; s < 8; ++s) {
                const uint32_t hb = s >= 2 ? (h >> (s - 2)) : (h << (2 - s));
                D[s] |= hb & 0x04040404u;
            }
        }
    } else if constexpr (BITS == 4) {
        const u4& u = r.c[tau];
#pragma unroll
        for (int m = 0; m < 4; ++m) {
            const uint32_t w = wsel(u, m);
            D[2 * m] = w & 0x0F0F0F0Fu;
            D[2 * m + 1] = (w >> 4) & 0x0F0F0F0Fu;
        }
    } else {
        const u4& a = r.c[2 * tau];
        const u4& b = r.c[2 * tau + 1];
        D[0] = a.x; D[1] = a.y; D[2] = a.z; D[3] = a.w;
        D[4] = b.x; D[5] = b.y; D[6] = b.z; D[7] = b.w;
    }
}

// f32(fp16 half `hi` of `packed`) * x with one rounding (v_fma_mix_f32 with addend -0: exactly the fp32 product,
// including the sign of zero), i.e. the same value as converting the scale and multiplying
__device__ __forceinline__ float mul_f16_f32(uint32_t packed, int hi, float x) {
    float r;
    if (hi) asm("v_fma_mix_f32 %0, %1, %2, %3 op_sel:[1,0,0] op_sel_hi:[1,0,0]" : "=v"(r) : "v"(packed), "v"(x), "v"(-0.0f));
    else asm("v_fma_mix_f32 %0, %1, %2, %3 op_sel_hi:[1,0,0]" : "=v"(r) : "v"(packed), "v"(x), "v"(-0.0f));
    return r;
}

// packlib strip row of device gate_up strip row d (inverse of the interleave written by relayout.hip)
__device__ __forceinline__ int gu_packlib_row(int d) {
    const int q = d >> 2, v = d & 3;
    return (v & 1) ? 8 + 2 * q + (v >> 1) : 2 * q + (v >> 1);
}

template <int MODE>
struct Geo {
    static constexpr bool DOWN_SHAPE = MODE == GEMM_DOWN || MODE == GEMM_PRODUCTS_DOWN;
    static constexpr bool PRODUCTS = MODE == GEMM_PRODUCTS_GATE_UP || MODE == GEMM_PRODUCTS_DOWN;
    static constexpr int NSB = DOWN_SHAPE ? 1 : 4;       // K = 512 or 2048
    // strips per wave (streamed as one ring) by code width, so that every wave streams about the same bytes
    // (~35 KB): the workgroups of wide codes would otherwise be the tail of the launch
    template <int BITS>
    static constexpr int spw() { return gemm_spw(DOWN_SHAPE, BITS); }
    static constexpr int SPW_MAX = spw<2>();
};

// ring depth (superblock steps in flight per wave), a divisor of 4: a wave keeps 4 steps -- 8 to 16 KiB -- in
// flight (2 of 8-bit codes). The layer GEMMs are built for 3 waves per SIMD (168 VGPRs): measured at 32 tokens
// against 2 (gate_up 32.0 -> 29.1 us) and 4 (which needs a ring of 2 steps and spills: 30.7 us, down 17.5 ->
// 20.4 us).
template <int BITS>
struct Ring {
    static constexpr int D = BITS == 8 ? 2 : 4;
};

// LDS: B rows [ntok][K + 16], B scales and sums [K/128][ntok] x 2, then one 192-byte meta slot per wave (the
// current superblock's scales and zeros, written from the ring and read back per lane quad)
__host__ __device__ constexpr int b_bytes(int ntok, int K) { return ntok * (K + 16) + ntok * (K / GROUP) * 8; }
template <int MODE>
__host__ __device__ constexpr int meta_bytes() { return WAVES * META_SB; }
// the down GEMM's slot outputs of one unit, buffered in LDS and stored after the weight stream when they fit: up to
// 4 tokens of a 2-bit unit (1024 rows), 8 of 3/4-bit (512), 16 of 8-bit (256)
constexpr int YBUF_BYTES = 16384;
template <int MODE, int NT>
__host__ __device__ constexpr int ybuf_offset() {
    return b_bytes(16 * NT, Geo<MODE>::NSB * SB_K) + meta_bytes<MODE>() + 16 * NT * 4;   // + the B row table
}
// the gate_up GEMM's Z outputs of one unit (at most 16 tokens x 128 fp16)
constexpr int ZBUF_BYTES = 16 * 128 * 2;
template <int MODE, int NT>
__host__ __device__ constexpr int lds_bytes() {
    return ybuf_offset<MODE, NT>() + (MODE == GEMM_DOWN && NT == 1 ? YBUF_BYTES : 0) +
           (MODE == GEMM_GATE_UP && NT == 1 ? ZBUF_BYTES : 0);
}

// the plan of a self-planning decode gate_up GEMM: the unit's token rows come from its token masks
struct RowSrc {
    const DecodePlan* P;
    int T, K, E;
};

template <int BITS, int MODE, int NT, bool PLAN = false>
__device__ __forceinline__ void gemm_body(const GemmArgs& a, const Item& it, const uint8_t* mat_e, uint8_t* lds,
                                          int row_block, const RowSrc& rs = RowSrc{}) {
    constexpr int NSB = Geo<MODE>::NSB, SPW = Geo<MODE>::template spw<BITS>(), NSTEP = NSB * SPW;
    constexpr int D = Ring<BITS>::D < NSTEP ? Ring<BITS>::D : NSTEP;
    static_assert(NSTEP % 4 == 0 && 4 % D == 0, "ring geometry");
    constexpr int K = NSB * SB_K, G = K / GROUP, NTOK = 16 * NT, LDQ = K + 16;
    constexpr size_t SBB = sb_bytes(BITS);
    constexpr int ZOFF = BITS == 8 ? 128 : 0;
    // (the thread index made opaque: values derived from it are recomputed per unit, not kept live -- and
    // spilled -- across the unit loop)
    int tid = threadIdx.x;
    asm volatile("" : "+v"(tid));
    const int lane = tid & 63, wave = tid >> 6, q = lane >> 4, col = lane & 15;
    if ((row_block + 1) * WAVES * SPW * 16 > a.R) return;    // not a row block of this code width
    // the row block's strips interleaved over the waves (wave w takes strips w, w + WAVES, ...): at each step the
    // workgroup's waves read adjacent superblocks (config 1: 0.0566 -> 0.0559 ms against contiguous strips per wave)
    const int sbase = row_block * WAVES * SPW;
    auto step_ptr = [&](int u) { return mat_e + (size_t(sbase + (u / NSB) * WAVES + wave) * NSB + (u % NSB)) * SBB; };

    // weight prefetch first: its latency overlaps the meta and B staging below (the down GEMM's Z rows, whose
    // addresses need no load, are requested before it, so their transform overlaps the ring fill)
    Step<BITS> ring[D];
    constexpr bool ZIN = MODE == GEMM_DOWN;
    constexpr int PERW = NTOK / WAVES;
    uint4 zraw[ZIN ? PERW : 1];
    if (ZIN && a.zin != nullptr) {
#pragma unroll
        for (int i = 0; i < PERW; ++i) {
            const int n = wave + i * WAVES;
            zraw[i] = n < it.ntok ? *reinterpret_cast<const uint4*>(a.zin + size_t(it.slot0 + n) * K + 8 * lane)
                                  : make_uint4(0u, 0u, 0u, 0u);
        }
    }
#pragma unroll
    for (int u = 0; u < D; ++u)
        if (u < NSTEP) load_step<BITS>(step_ptr(u), lane, ring[u]);

    // this wave's meta slot
    uint8_t* meta_lds = lds + b_bytes(NTOK, K);
    uint8_t* mp = meta_lds + wave * META_SB;

    // stage the item's B rows in LDS: q8 rows [NTOK][LDQ], scales [G][NTOK], sums [G][NTOK]
    int8_t* bq = reinterpret_cast<int8_t*>(lds);
    float* bs = reinterpret_cast<float*>(lds + NTOK * LDQ);
    int* bsum = reinterpret_cast<int*>(bs + G * NTOK);
    const int ntok = it.ntok;
    if (MODE == GEMM_DOWN && a.zin != nullptr) {
        // B rows = A8(FWHT-512(Z)) of the item's slots, slot n on wave n % WAVES (the operations of
        // fwht_a8_kernel); the units of row block 0 also store them for the buffers' readers. Rows n >= ntok are
        // zero. The wave's Z rows are all loaded before the first transform, so their latencies overlap.
        static_assert(PERW * WAVES == NTOK, "slots per wave");
#pragma unroll
        for (int i = 0; i < PERW; ++i) {
            const int n = wave + i * WAVES;
            uint2 qw = make_uint2(0u, 0u);
            float sc = 0.0f;
            int tot = 0;
            if (n < ntok) {
                const size_t slot = size_t(it.slot0 + n);
                fwht512_a8_raw(zraw[i], lane, qw, sc, tot);
                if (row_block == 0) {
                    *reinterpret_cast<uint2*>(a.xq_out + slot * K + 8 * lane) = qw;
                    if ((lane & 15) == 0) {
                        a.xs_out[slot * G + (lane >> 4)] = sc;
                        a.xsum_out[slot * G + (lane >> 4)] = tot;
                    }
                }
            }
            *reinterpret_cast<uint2*>(bq + n * LDQ + 8 * lane) = qw;
            if ((lane & 15) == 0) {
                bs[(lane >> 4) * NTOK + n] = sc;
                bsum[(lane >> 4) * NTOK + n] = -tot;   // negated: C = zero * (-sum)
            }
        }
    } else {
        // B rows through a row table in LDS (one round of slot_token loads), then NTOK * K / 16 chunks of 16
        // bytes over 256 threads at clamped rows, all issued before the LDS stores
        int* rowtab = reinterpret_cast<int*>(meta_lds + meta_bytes<MODE>());
        if (threadIdx.x < NTOK) {
            const int n = min(int(threadIdx.x), ntok - 1), slot = it.slot0 + n;
            if constexpr (PLAN) rowtab[threadIdx.x] = decode_slot_token(*rs.P, it, n, rs.T, rs.K, rs.E);
            else rowtab[threadIdx.x] = a.slot_token ? a.slot_token[slot] : slot;
        }
        __syncthreads();
        constexpr int CH = K / 16, PER = (NTOK * CH + WAVES * 64 - 1) / (WAVES * 64);
        u4 v[PER];
#pragma unroll
        for (int i = 0; i < PER; ++i) {
            const int idx = threadIdx.x + i * WAVES * 64, c16 = idx % CH;
            v[i] = *reinterpret_cast<const u4*>(a.xq + size_t(rowtab[min(idx / CH, NTOK - 1)]) * K + 16 * c16);
        }
        constexpr int PG = (NTOK * G + WAVES * 64 - 1) / (WAVES * 64);
        float sv[PG];
        int qv[PG];
#pragma unroll
        for (int i = 0; i < PG; ++i) {
            const int idx = threadIdx.x + i * WAVES * 64, g = idx % G;
            const size_t row = size_t(rowtab[min(idx / G, NTOK - 1)]);
            sv[i] = a.xs ? a.xs[row * G + g] : 0.0f;
            qv[i] = a.xsum[row * G + g];
        }
        // rows n >= ntok are zero: the MFMA columns of absent tokens then compute zeros, branch-free
#pragma unroll
        for (int i = 0; i < PER; ++i) {
            const int idx = threadIdx.x + i * WAVES * 64, n = idx / CH, c16 = idx % CH;
            if (n < NTOK) *reinterpret_cast<u4*>(bq + n * LDQ + 16 * c16) = n < ntok ? v[i] : u4{0u, 0u, 0u, 0u};
        }
#pragma unroll
        for (int i = 0; i < PG; ++i) {
            const int idx = threadIdx.x + i * WAVES * 64, n = idx / G, g = idx % G;
            if (n < NTOK) {
                bs[g * NTOK + n] = n < ntok ? sv[i] : 0.0f;
                bsum[g * NTOK + n] = n < ntok ? -qv[i] : 0;          // negated: C = zero * (-sum)
            }
        }
    }
    __syncthreads();

    // routing weights of this lane's slots, read before the stream: a load inside the ring would make the
    // compiler wait for every outstanding weight load
    float wts[NT];
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
        const int n = nt * 16 + col;
        wts[nt] = (MODE == GEMM_DOWN && n < ntok) ? a.slot_weight[it.slot0 + n] : 0.0f;
    }
    float acc[NT][4];
#pragma unroll
    for (int nt = 0; nt < NT; ++nt)
#pragma unroll
        for (int v = 0; v < 4; ++v) acc[nt][v] = 0.0f;
    // down: the unit's outputs w acc go to LDS ([slot][row of the unit]) and are stored after the stream, in one
    // coalesced pass, when they fit: the partial-wave stores of one or a few tokens inside the stream slow it
    // (config 1: 0.0553 -> 0.0549 ms per step; config 0, whose equal 4-bit units all end with the pass, 0.0431 ->
    // 0.0433 ms)
    constexpr int UROWS = WAVES * SPW * 16;
    const bool ybuf = MODE == GEMM_DOWN && NT == 1 && ntok * UROWS * 4 <= YBUF_BYTES;
    float* ylds = reinterpret_cast<float*>(lds + ybuf_offset<MODE, NT>());
    // gate_up: the same for Z ([slot][UROWS / 2] fp16), which always fits; the partial-wave Z stores inside the
    // stream cost up to 0.67 us of the config-1 step (a diagnostic build without them)
    constexpr bool ZBUF = MODE == GEMM_GATE_UP && NT == 1;
    static_assert(!ZBUF || UROWS / 2 * 16 * 2 <= ZBUF_BYTES, "Z buffer");
    uint32_t* zlds = reinterpret_cast<uint32_t*>(lds + ybuf_offset<MODE, NT>());

    // the wave's NSTEP superblocks (SPW strips of NSB each) are streamed as one ring (slot of step u = u % D). The steps are unrolled at compile time: across a loop back-edge the compiler would wait for every
    // outstanding load, and the prefetch would not overlap.
    static_for<0, NSTEP>([&](auto uc) {
        constexpr int u = decltype(uc)::value;
        Step<BITS>& cur = ring[u % D];
        constexpr int sb = u % NSB;
        const int strip = sbase + (u / NSB) * WAVES + wave;
        // the wave's meta slot: lanes 0-47 store the superblock's 192 bytes, then every lane reads other lanes'
        // bytes. A wave's LDS operations execute in program order; the wave barriers keep the compiler from moving
        // this step's store above the previous step's reads or the reads above the store.
        __builtin_amdgcn_wave_barrier();
        if (lane < META_SB / 4) *reinterpret_cast<uint32_t*>(mp + 4 * lane) = cur.m;
        __builtin_amdgcn_wave_barrier();
        const u4 ms0 = *reinterpret_cast<const u4*>(mp + 32 * q);
        const u4 ms1 = *reinterpret_cast<const u4*>(mp + 32 * q + 16);
        const u4 zw4 = *reinterpret_cast<const u4*>(mp + 128 + 16 * q);
        if constexpr (!Geo<MODE>::PRODUCTS && NT == 1) {
            // layer GEMMs (one token tile): software-pipelined over the 4 tiles, the MFMAs of tile tau issued
            // before the fp32 epilogue of tile tau - 1, so the MFMA latency overlaps vector work
            v4i Cp;
            float xsp = 0.0f;
            uint32_t swpp[2] = {0u, 0u};
            static_for<0, 5>([&](auto tc) {
                constexpr int tau = decltype(tc)::value;
                v4i Cc;
                float xsc = 0.0f;
                uint32_t swc[2] = {0u, 0u};
                if constexpr (tau < 4) {
                    constexpr int g = sb * 4 + tau;
                    uint32_t Dw[8];
                    unpack_tile<BITS>(cur, tau, Dw);
                    const v4i A0 = {int(Dw[0]), int(Dw[1]), int(Dw[2]), int(Dw[3])};
                    const v4i A1 = {int(Dw[4]), int(Dw[5]), int(Dw[6]), int(Dw[7])};
                    const uint32_t zw = zw4[tau];
                    const u4& sv = tau < 2 ? ms0 : ms1;
                    swc[0] = wsel(sv, (tau & 1) * 2);
                    swc[1] = wsel(sv, (tau & 1) * 2 + 1);
                    int zz[4];
#pragma unroll
                    for (int v = 0; v < 4; ++v) zz[v] = int((zw >> (8 * v)) & 0xFFu) - ZOFF;
                    const int8_t* br = bq + col * LDQ + g * GROUP + 16 * q;
                    const v4i B0 = *reinterpret_cast<const v4i*>(br);
                    const v4i B1 = *reinterpret_cast<const v4i*>(br + 64);
                    xsc = bs[g * NTOK + col];
                    const int nxsum = bsum[g * NTOK + col];
                    Cc = v4i{__mul24(zz[0], nxsum) + I2F_BIAS, __mul24(zz[1], nxsum) + I2F_BIAS,
                             __mul24(zz[2], nxsum) + I2F_BIAS, __mul24(zz[3], nxsum) + I2F_BIAS};
                    Cc = __builtin_amdgcn_mfma_i32_16x16x64_i8(A0, B0, Cc, 0, 0, 0);
                    Cc = __builtin_amdgcn_mfma_i32_16x16x64_i8(A1, B1, Cc, 0, 0, 0);
                }
                if constexpr (tau > 0) {
#pragma unroll
                    for (int v = 0; v < 4; ++v)
                        acc[0][v] = __builtin_fmaf(mul_f16_f32(swpp[v >> 1], v & 1, xsp), biased_to_f32(Cp[v]), acc[0][v]);
                    asm volatile("" : "+v"(acc[0][0]), "+v"(acc[0][1]), "+v"(acc[0][2]), "+v"(acc[0][3]));
                }
                if constexpr (tau < 4) {
                    Cp = Cc;
                    xsp = xsc;
                    swpp[0] = swc[0];
                    swpp[1] = swc[1];
                }
                __builtin_amdgcn_sched_barrier(0);
            });
        } else {
    #pragma unroll
            for (int tau = 0; tau < 4; ++tau) {
                const int g = sb * 4 + tau;
                uint32_t Dw[8];
                unpack_tile<BITS>(cur, tau, Dw);
                const v4i A0 = {int(Dw[0]), int(Dw[1]), int(Dw[2]), int(Dw[3])};
                const v4i A1 = {int(Dw[4]), int(Dw[5]), int(Dw[6]), int(Dw[7])};
                const uint32_t zw = zw4[tau];
                const u4& sv = tau < 2 ? ms0 : ms1;
                const uint32_t s01 = wsel(sv, (tau & 1) * 2), s23 = wsel(sv, (tau & 1) * 2 + 1);
                const uint32_t swp[2] = {s01, s23};   // fp16 scale pairs (rows 4q + 0, 1 | 2, 3)
                int zz[4];
    #pragma unroll
                for (int v = 0; v < 4; ++v) zz[v] = int((zw >> (8 * v)) & 0xFFu) - ZOFF;
    #pragma unroll
                for (int nt = 0; nt < NT; ++nt) {
                    const int n = nt * 16 + col;
                    const int8_t* br = bq + n * LDQ + g * GROUP + 16 * q;
                    const v4i B0 = *reinterpret_cast<const v4i*>(br);
                    const v4i B1 = *reinterpret_cast<const v4i*>(br + 64);
                    const float xsn = bs[g * NTOK + n];
                    const int nxsum = bsum[g * NTOK + n];
                    v4i C = {__mul24(zz[0], nxsum), __mul24(zz[1], nxsum), __mul24(zz[2], nxsum), __mul24(zz[3], nxsum)};
                    C = __builtin_amdgcn_mfma_i32_16x16x64_i8(A0, B0, C, 0, 0, 0);
                    C = __builtin_amdgcn_mfma_i32_16x16x64_i8(A1, B1, C, 0, 0, 0);
                    if constexpr (Geo<MODE>::PRODUCTS) {
                        if (n < ntok) {
    #pragma unroll
                            for (int v = 0; v < 4; ++v) {
                                const int d = 4 * q + v;
                                const int prow = 16 * strip + (MODE == GEMM_PRODUCTS_GATE_UP ? gu_packlib_row(d) : d);
                                a.P[(size_t(it.slot0 + n) * a.R + prow) * G + g] = C[v];
                            }
                        }
                    } else {
    #pragma unroll
                        for (int v = 0; v < 4; ++v)
                            acc[nt][v] = __builtin_fmaf(mul_f16_f32(swp[v >> 1], v & 1, xsn), float(C[v]), acc[nt][v]);
                    }
                }
                // one tile at a time: the accumulators are materialised here, otherwise the compiler defers each
                // tile's fp32 accumulation (a serial fma chain) to the strip end and keeps every tile's results live
                if constexpr (!Geo<MODE>::PRODUCTS) {
    #pragma unroll
                    for (int nt = 0; nt < NT; ++nt)
                        asm volatile("" : "+v"(acc[nt][0]), "+v"(acc[nt][1]), "+v"(acc[nt][2]), "+v"(acc[nt][3]));
                }
                __builtin_amdgcn_sched_barrier(0);
            }
        }
        if constexpr (!Geo<MODE>::PRODUCTS && sb == NSB - 1) {   // strip done: fused epilogue
#pragma unroll
            for (int nt = 0; nt < NT; ++nt) {
                const int n = nt * 16 + col;
                if (n < ntok) {
                    const int slot = it.slot0 + n;
                    if constexpr (MODE == GEMM_GATE_UP) {
                        // lane quad q holds rows gate 8 strip + 2q, up (same), gate + 1, up + 1
                        uint32_t z0, z1;
                        if (a.fast) {
                            z0 = silu_mul_f16_fast(acc[nt][0], acc[nt][1]);
                            z1 = silu_mul_f16_fast(acc[nt][2], acc[nt][3]);
                        } else {
                            z0 = f32_to_f16_rne(silu_f32(acc[nt][0]) * acc[nt][1]);
                            z1 = f32_to_f16_rne(silu_f32(acc[nt][2]) * acc[nt][3]);
                        }
                        if constexpr (ZBUF) zlds[n * (UROWS / 4) + 4 * (strip - sbase) + q] = z0 | (z1 << 16);
                        else *reinterpret_cast<uint32_t*>(a.Z + size_t(slot) * (a.R / 2) + 8 * strip + 2 * q) = z0 | (z1 << 16);
                    } else if (ybuf) {
                        *reinterpret_cast<float4*>(ylds + n * UROWS + 16 * (strip - sbase) + 4 * q) =
                            make_float4(wts[nt] * acc[nt][0], wts[nt] * acc[nt][1], wts[nt] * acc[nt][2],
                                        wts[nt] * acc[nt][3]);
                    } else {
                        store_slot_out(a, size_t(slot) * a.R + 16 * strip + 4 * q, wts[nt], acc[nt][0], acc[nt][1],
                                       acc[nt][2], acc[nt][3]);
                    }
                }
#pragma unroll
                for (int v = 0; v < 4; ++v) acc[nt][v] = 0.0f;
            }
        }
        // refill the slot just consumed with step u + D
        if constexpr (u + D < NSTEP) load_step<BITS>(step_ptr(u + D), lane, cur);
    });
    if constexpr (ZBUF) {
        // the wave stores the Z it wrote (its strips j WAVES + wave, 16 bytes each per slot), one store per lane
        // and no workgroup barrier (config 1: 0.0549 -> 0.0544 ms per step; through a barrier and a workgroup-wide
        // pass: 0.0546)
        static_assert(16 * Geo<MODE>::SPW_MAX <= 64, "one store per lane");
        __builtin_amdgcn_wave_barrier();
        if (lane < ntok * SPW) {
            const int n = lane / SPW, c = (lane % SPW) * WAVES + wave;
            *reinterpret_cast<uint4*>(a.Z + size_t(it.slot0 + n) * (a.R / 2) + 8 * (sbase + c)) =
                *reinterpret_cast<const uint4*>(zlds + n * (UROWS / 4) + 4 * c);
        }
    }
    if constexpr (MODE == GEMM_DOWN && NT == 1) {
        if (ybuf) {
            __syncthreads();
            // each slot's UROWS outputs are contiguous in Y (rows 16 sbase ...), 16 bytes per thread
            for (int idx = tid; idx < ntok * (UROWS / 4); idx += WAVES * 64) {
                const int n = idx / (UROWS / 4), r4 = idx % (UROWS / 4);
                const float4 y = *reinterpret_cast<const float4*>(ylds + 4 * idx);
                store_slot_out(a, size_t(it.slot0 + n) * a.R + 16 * sbase + 4 * r4, 1.0f, y.x, y.y, y.z, y.w);
            }
        }
    }
}

// Persistent: the grid is the number of workgroups that fit the GPU at once; each workgroup takes the work units
// blockIdx.x, blockIdx.x + gridDim.x, ... (units are ordered longest first, so the long ones start first).
// Measured at 32 tokens and not kept: units claimed from a device counter as workgroups become free (0.0625 ->
// 0.073 ms per step: same-address device-scope atomics serialise across the 8 XCDs), and a second round assigned
// in reverse (0.0610 -> 0.0631 ms).
template <int MODE, int NT>
__global__ void __launch_bounds__(WAVES * 64, NT == 1 ? 3 : 1) expert_gemm(GemmArgs a) {
    extern __shared__ __align__(16) uint8_t lds[];
    if (MODE == GEMM_DOWN && a.clear_a != nullptr && blockIdx.x == 0)
        for (int i = threadIdx.x; i < a.nclear; i += blockDim.x) {
            a.clear_a[i] = 0u;
            a.clear_b[i] = 0u;
        }
    // the unit and the expert's code width and matrix offset are read through the scalar cache (constant address
    // space: the lists are written by earlier kernels only), the width and offset together, so the weight stream
    // starts after two short dependent loads
    const int n = *a.n_items;
    for (int u = blockIdx.x; u < n; u += gridDim.x) {
        const auto* ip = const_ptr(reinterpret_cast<const int*>(a.items + u));
        const Item it{ip[0], ip[1], ip[2], ip[3]};
        const uint64_t off = *const_ptr(a.off + it.expert);
        const uint32_t bw4 = *const_ptr(reinterpret_cast<const uint32_t*>(a.bits) + (it.expert >> 2));
        asm volatile("" ::"s"(off), "s"(bw4));   // both loads in flight together, before the branch on the width
        const int bits = int(bw4 >> (8 * (it.expert & 3))) << 24 >> 24;
        const uint8_t* mat_e = a.base + off;
        if (bits == 2) gemm_body<2, MODE, NT>(a, it, mat_e, lds, it.rb);
        else if (bits == 3) gemm_body<3, MODE, NT>(a, it, mat_e, lds, it.rb);
        else if (bits == 4) gemm_body<4, MODE, NT>(a, it, mat_e, lds, it.rb);
        else gemm_body<8, MODE, NT>(a, it, mat_e, lds, it.rb);
        __syncthreads();   // the next unit re-stages the LDS
    }
}

// The decode gate_up GEMM of a layer forward, planning for itself: every workgroup builds the slot plan in LDS from
// the routing masks (decode_plan.h) and takes the units blockIdx.x, blockIdx.x + gridDim.x, ... of the gate_up list
// that the dispatch kernel would have written; workgroups G - 1 - r, r = 0 .. E, write the plan's lists first (expert
// r's units, or the shared units and the placement), for the down GEMM, the combine and the buffers' readers, and a
// copy of the masks (tcopy) from which a re-launch plans the same units after the down GEMM has zeroed them.
__global__ void __launch_bounds__(WAVES * 64, 3) expert_gemm_plan(GemmArgs a, DecodePlanArgs p) {
    extern __shared__ __align__(16) uint8_t lds[];
    __shared__ DecodePlan P;
    decode_plan_scan(p.E, p.tmask, p.d.bits, P);
    const int sbits = p.d.has_shared ? p.d.bits[p.E] : 8;
    // the writer roles go to the last workgroups, whose units are in the first round only (config 1: 56.8 -> 56.2 us
    // against the first workgroups)
    for (int r = int(gridDim.x - 1 - blockIdx.x); r <= p.E; r += gridDim.x) {
        if (r < p.E) {
            decode_plan_write_expert(P, r, threadIdx.x, blockDim.x, p.d);
        } else {
            decode_plan_write_rest(P, threadIdx.x, blockDim.x, p.T, p.E, p.K, p.topk, p.topw, p.d);
            if (threadIdx.x < p.E) p.tcopy[threadIdx.x] = P.m[threadIdx.x];
        }
    }
    const int n = decode_plan_units(P, false, p.T, p.d.has_shared, sbits);
    const RowSrc rs{&P, p.T, p.K, p.E};
    for (int u = blockIdx.x; u < n; u += gridDim.x) {
        const Item q = decode_plan_unit(P, false, u, p.T, p.E, p.K, sbits);
        const Item it{__builtin_amdgcn_readfirstlane(q.expert), __builtin_amdgcn_readfirstlane(q.slot0),
                      __builtin_amdgcn_readfirstlane(q.ntok), __builtin_amdgcn_readfirstlane(q.rb)};
        const uint64_t off = *const_ptr(a.off + it.expert);
        const int bits = it.expert < p.E ? __builtin_amdgcn_readfirstlane(int(P.bits[it.expert])) : sbits;
        const uint8_t* mat_e = a.base + off;
        if (bits == 2) gemm_body<2, GEMM_GATE_UP, 1, true>(a, it, mat_e, lds, it.rb, rs);
        else if (bits == 3) gemm_body<3, GEMM_GATE_UP, 1, true>(a, it, mat_e, lds, it.rb, rs);
        else if (bits == 4) gemm_body<4, GEMM_GATE_UP, 1, true>(a, it, mat_e, lds, it.rb, rs);
        else gemm_body<8, GEMM_GATE_UP, 1, true>(a, it, mat_e, lds, it.rb, rs);
        __syncthreads();   // the next unit re-stages the LDS
    }
    // When the gate_up units fit one round, every workgroup then requests the first pf_bytes of down units
    // blockIdx.x, blockIdx.x + G, ... (one dword per 64-byte line), so that the down GEMM finds them in the
    // last-level cache (config 0: 0.0429 -> 0.0419 ms per step with 48 KiB; 96 KiB and more slow gate_up down).
    // With a second gate_up round the same requests take bandwidth from it: config 1 (908 units on 768
    // workgroups) went from 0.0540 to 0.0551 ms with 16 KiB requested by the single-unit workgroups.
    const int G = int(gridDim.x);
    if (p.pf_bytes > 0 && n <= G) {
        const int ndn = decode_plan_units(P, true, p.T, p.d.has_shared, sbits);
        uint32_t sink = 0u;
        for (int d = int(blockIdx.x); d < ndn; d += G) {
            const Item q = decode_plan_unit(P, true, d, p.T, p.E, p.K, sbits);
            const int e = __builtin_amdgcn_readfirstlane(q.expert), rb = __builtin_amdgcn_readfirstlane(q.rb);
            const int bits = e < p.E ? __builtin_amdgcn_readfirstlane(int(P.bits[e])) : sbits;
            const int ub = GEMM_WAVES * gemm_spw(true, bits) * int(sb_bytes(bits)), len = min(ub, p.pf_bytes);
            const uint8_t* src = a.base + *const_ptr(p.d_off + e) + size_t(rb) * ub;
#pragma unroll 8
            for (int i = int(threadIdx.x) * 64; i < len; i += int(blockDim.x) * 64)
                sink ^= *reinterpret_cast<const uint32_t*>(src + i);
        }
        asm volatile("" ::"v"(sink));
    }
}

// Dense projection at T <= 32, split over K: workgroup (strip s, token tiles) computes 16 rows x 16 NTL tokens;
// wave w loads only superblock w of the strip (groups 4w .. 4w + 3), with its B operands straight from x' (a few KiB,
// resident in L2). Its exact group products P_g (the biased accumulator's float) and scale products sw sx go through
// LDS; then wave v accumulates value v of every lane (rows 4q + v) over the 16 groups in ascending order: the fp32
// sequence of the streamed GEMM, with four waves in flight per strip (NTL 16-token tiles per workgroup).
template <int NTL>
__host__ __device__ constexpr int dense_lds() { return NTL * 2 * 16 * 4 * 64 * 4 + WAVES * META_SB; }
template <int BITS, int NTL>
__global__ void __launch_bounds__(WAVES * 64) dense_splitk_kernel(GemmArgs a) {
    static_assert(WAVES == 4, "one superblock per wave");
    constexpr int G = 16;
    constexpr size_t SBB = sb_bytes(BITS);
    constexpr int ZOFF = BITS == 8 ? 128 : 0;
    extern __shared__ __align__(16) uint8_t dl[];
    float (*Ps)[G][4][64] = reinterpret_cast<float (*)[G][4][64]>(dl);                          // [NTL]
    float (*Ss)[G][4][64] = reinterpret_cast<float (*)[G][4][64]>(dl + NTL * G * 4 * 64 * 4);   // [NTL]
    uint8_t* meta = dl + 2 * NTL * G * 4 * 64 * 4;
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, q = lane >> 4, col = lane & 15;
    const int s = blockIdx.x, t0 = 16 * NTL * int(blockIdx.y);
    Step<BITS> st;
    load_step<BITS>(a.base + *const_ptr(a.off) + (size_t(s) * 4 + w) * SBB, lane, st);
    v4i B0[NTL][4], B1[NTL][4];
    float xsv[NTL][4];
    int nxs[NTL][4];
#pragma unroll
    for (int tt = 0; tt < NTL; ++tt) {
        // absent tokens read a present row; their outputs are not stored
        const int tok = min(t0 + 16 * tt + col, a.dense_T - 1);
#pragma unroll
        for (int tau = 0; tau < 4; ++tau) {
            const int g = 4 * w + tau;
            const int8_t* br = a.xq + size_t(tok) * 2048 + g * GROUP + 16 * q;
            B0[tt][tau] = *reinterpret_cast<const v4i*>(br);
            B1[tt][tau] = *reinterpret_cast<const v4i*>(br + 64);
            xsv[tt][tau] = a.xs[size_t(tok) * G + g];
            nxs[tt][tau] = -a.xsum[size_t(tok) * G + g];
        }
    }
    // the superblock's scales and zeros through the wave's LDS slot (as in gemm_body)
    uint8_t* mp = meta + w * META_SB;
    __builtin_amdgcn_wave_barrier();
    if (lane < META_SB / 4) *reinterpret_cast<uint32_t*>(mp + 4 * lane) = st.m;
    __builtin_amdgcn_wave_barrier();
    const u4 ms0 = *reinterpret_cast<const u4*>(mp + 32 * q);
    const u4 ms1 = *reinterpret_cast<const u4*>(mp + 32 * q + 16);
    const u4 zw4 = *reinterpret_cast<const u4*>(mp + 128 + 16 * q);
#pragma unroll
    for (int tau = 0; tau < 4; ++tau) {
        const int g = 4 * w + tau;
        uint32_t Dw[8];
        unpack_tile<BITS>(st, tau, Dw);
        const v4i A0 = {int(Dw[0]), int(Dw[1]), int(Dw[2]), int(Dw[3])};
        const v4i A1 = {int(Dw[4]), int(Dw[5]), int(Dw[6]), int(Dw[7])};
        const uint32_t zw = zw4[tau];
        const u4& sv = tau < 2 ? ms0 : ms1;
        const uint32_t swp[2] = {wsel(sv, (tau & 1) * 2), wsel(sv, (tau & 1) * 2 + 1)};
#pragma unroll
        for (int tt = 0; tt < NTL; ++tt) {
            v4i C;
#pragma unroll
            for (int v = 0; v < 4; ++v) C[v] = __mul24(int((zw >> (8 * v)) & 0xFFu) - ZOFF, nxs[tt][tau]) + I2F_BIAS;
            C = __builtin_amdgcn_mfma_i32_16x16x64_i8(A0, B0[tt][tau], C, 0, 0, 0);
            C = __builtin_amdgcn_mfma_i32_16x16x64_i8(A1, B1[tt][tau], C, 0, 0, 0);
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                Ps[tt][g][v][lane] = biased_to_f32(C[v]);
                Ss[tt][g][v][lane] = mul_f16_f32(swp[v >> 1], v & 1, xsv[tt][tau]);
            }
        }
    }
    __syncthreads();
#pragma unroll
    for (int tt = 0; tt < NTL; ++tt) {
        float acc = 0.0f;
#pragma unroll
        for (int g = 0; g < G; ++g) acc = __builtin_fmaf(Ss[tt][g][w][lane], Ps[tt][g][w][lane], acc);
        const int t = t0 + 16 * tt + col;
        if (t < a.dense_T) {
            float* yp = a.Y + size_t(t) * a.R + 16 * s + 4 * q + w;
            *yp = a.accumulate ? *yp + acc : acc;
        }
    }
}

template <int MODE, int NT>
const void* kernel_ptr() { return reinterpret_cast<const void*>(&expert_gemm<MODE, NT>); }

template <int MODE, int NT>
hipError_t set_attr() {
    constexpr int K = Geo<MODE>::NSB * SB_K;
    return hipFuncSetAttribute(kernel_ptr<MODE, NT>(), hipFuncAttributeMaxDynamicSharedMemorySize, lds_bytes<MODE, NT>());
}

template <int MODE, int NT>
hipError_t launch_t(const GemmArgs& a, int, hipStream_t st) {
    static int grid = 0;
    if (!grid) {   // workgroups resident at once on the whole GPU
        int dev = 0, cus = 0, per_cu = 0;
        hipError_t e = hipGetDevice(&dev);
        if (e == hipSuccess) e = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
        if (e == hipSuccess)
            e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kernel_ptr<MODE, NT>(), WAVES * 64,
                                                             lds_bytes<MODE, NT>());
        if (e != hipSuccess) return e;
        grid = cus * (per_cu > 0 ? per_cu : 1);
    }
    expert_gemm<MODE, NT><<<grid, WAVES * 64, lds_bytes<MODE, NT>(), st>>>(a);
    return hipGetLastError();
}

}  // namespace

hipError_t gemm_setup() {
    hipError_t e;
    if ((e = hipFuncSetAttribute(reinterpret_cast<const void*>(&expert_gemm_plan),
                                 hipFuncAttributeMaxDynamicSharedMemorySize, lds_bytes<GEMM_GATE_UP, 1>())) != hipSuccess)
        return e;
    if ((e = set_attr<GEMM_GATE_UP, 1>()) != hipSuccess) return e;
    if ((e = set_attr<GEMM_DOWN, 1>()) != hipSuccess) return e;
    if ((e = set_attr<GEMM_PRODUCTS_GATE_UP, 4>()) != hipSuccess) return e;
    if ((e = set_attr<GEMM_PRODUCTS_DOWN, 4>()) != hipSuccess) return e;
    return hipSuccess;
}

hipError_t launch_expert_gemm_plan(const GemmArgs& a, const DecodePlanArgs& p, hipStream_t st) {
    if (p.T < 1 || p.T > 32 || p.E < 1 || p.E > PLAN_MAXE) return hipErrorInvalidValue;
    static int grid = 0;
    if (!grid) {   // workgroups resident at once on the whole GPU
        int dev = 0, cus = 0, per_cu = 0;
        hipError_t e = hipGetDevice(&dev);
        if (e == hipSuccess) e = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
        if (e == hipSuccess)
            e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, reinterpret_cast<const void*>(&expert_gemm_plan),
                                                             WAVES * 64, lds_bytes<GEMM_GATE_UP, 1>());
        if (e != hipSuccess) return e;
        grid = cus * (per_cu > 0 ? per_cu : 1);
    }
    expert_gemm_plan<<<grid, WAVES * 64, lds_bytes<GEMM_GATE_UP, 1>(), st>>>(a, p);
    return hipGetLastError();
}

template <int NTL>
hipError_t dense_splitk_t(int bits, const GemmArgs& a, hipStream_t st) {
    static bool attr = false;
    if (!attr) {   // (above the default 64 KiB of LDS from two tiles on)
        hipError_t e = hipSuccess;
        for (const void* k : {reinterpret_cast<const void*>(&dense_splitk_kernel<2, NTL>),
                              reinterpret_cast<const void*>(&dense_splitk_kernel<3, NTL>),
                              reinterpret_cast<const void*>(&dense_splitk_kernel<4, NTL>),
                              reinterpret_cast<const void*>(&dense_splitk_kernel<8, NTL>)})
            if (e == hipSuccess) e = hipFuncSetAttribute(k, hipFuncAttributeMaxDynamicSharedMemorySize, dense_lds<NTL>());
        if (e != hipSuccess) return e;
        attr = true;
    }
    const dim3 grid(a.R / 16, (a.dense_T + 16 * NTL - 1) / (16 * NTL));
    constexpr int L = dense_lds<NTL>();
    if (bits == 2) dense_splitk_kernel<2, NTL><<<grid, WAVES * 64, L, st>>>(a);
    else if (bits == 3) dense_splitk_kernel<3, NTL><<<grid, WAVES * 64, L, st>>>(a);
    else if (bits == 4) dense_splitk_kernel<4, NTL><<<grid, WAVES * 64, L, st>>>(a);
    else if (bits == 8) dense_splitk_kernel<8, NTL><<<grid, WAVES * 64, L, st>>>(a);
    else return hipErrorInvalidValue;
    return hipGetLastError();
}

hipError_t launch_dense_splitk(int bits, const GemmArgs& a, hipStream_t st) {
    if (a.dense_T < 1 || a.dense_T > 32 || a.R % 16 || a.K != 2048) return hipErrorInvalidValue;
    // one 16-token tile per workgroup: two tiles per workgroup (the strip read once for 32 tokens, half the
    // workgroups, 66 KiB of LDS) measured 6.5 against 5.1 us at T = 32, [3072 x 2048]
    return dense_splitk_t<1>(bits, a, st);
}

// mode: GemmMode; nt: 16-token tiles per work item, 1 for the layer GEMMs (experts with many tokens take the
// tiled kernel), 4 for the products modes.
hipError_t launch_expert_gemm(int mode, int nt, const GemmArgs& a, int max_items, hipStream_t st) {
    if (mode == GEMM_GATE_UP) return nt == 1 ? launch_t<GEMM_GATE_UP, 1>(a, max_items, st) : hipErrorInvalidValue;
    if (mode == GEMM_DOWN) return nt == 1 ? launch_t<GEMM_DOWN, 1>(a, max_items, st) : hipErrorInvalidValue;
    if (mode == GEMM_PRODUCTS_GATE_UP) return launch_t<GEMM_PRODUCTS_GATE_UP, 4>(a, max_items, st);
    return launch_t<GEMM_PRODUCTS_DOWN, 4>(a, max_items, st);
}

}  // namespace llmoe
