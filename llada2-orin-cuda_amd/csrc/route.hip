// Router and dispatch kernels (engine/ops.cu:137-423): router logits, per-block sigmoid+bias scoring with the
// block expert pool and per-token top-K, routing weights, and the deterministic counting sort of (token, k)
// pairs into expert-major slots with the GEMM work items. All counts stay on the device.
#include "decode_plan.h"

namespace llmoe {

namespace {

constexpr int MAXB = 32;    // tokens per routing block (one 32-bit token mask per expert)
constexpr int MAXE = 256;   // experts (one thread each)
constexpr int PLAN_NT = 1024;          // planner threads: 4 per expert
constexpr int MAXB_BLOCKS = 128;       // routing blocks whose masks the planner holds in registers (32 per thread)

// logits partial c: fma chain over k = c H/8 .. (c+1) H/8 - 1 ascending from 0 (the summation order is fixed so
// the CPU checker reproduces it). Workgroup tile: TT tokens x EW experts of one K chunk, the chunk's x slice and
// its Wr slice (transposed, k contiguous per expert) staged in LDS, KS of k at a time; each thread runs one chain
// per (token, expert) it owns. grid (E/EW, ceil(T/TT), 8).
// With q != nullptr the workgroups also write the A8 of the x slice (two 128-groups per token, the same operations
// as quant_a8_kernel, spread over the expert slices), so the layer input is quantised without a launch of its own.
__device__ __forceinline__ uint32_t okey(float v) {        // order-preserving unsigned image of a float
    const uint32_t u = __float_as_uint(v);
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

constexpr int RKW = 256;                                          // K per chunk (H = 2048)
template <int KS>
constexpr int router_stride() { return KS + 4; }                  // LDS row stride of the x and Wr slices
template <int TT, int EW, int KS>
constexpr int router_lds() { return (TT + EW) * router_stride<KS>() * 4; }
// Tiles: <32 tokens, 8 experts, 256 threads> (one chain per thread: the decode step, latency-bound) and
// <64 tokens, 64 experts, 512 threads> (2 tokens x 4 experts per thread: x and Wr reloaded 8x less from L2). The
// chunk's K is staged KS at a time (the chains continue across the sub-chunks, so the order is the chunk's k
// ascending either way): KS = 128 keeps the large tile's LDS at 66 KiB, two workgroups per CU (at 512 tokens
// 20.0 -> 19.4 us per router stage, at 2048 tokens 66 -> 53 us, against one 133 KiB stage of 256 k). 4 tokens x 4
// experts per thread (half the LDS reads per fma, one wave per SIMD) measured 23 us at 512 tokens.
template <int TT, int EW, int NT, int TPT, int KS>
__global__ void __launch_bounds__(NT) router_logits_kernel(const float* __restrict__ x, const float* __restrict__ Wr,
                                                           int T, int H, int E, float* __restrict__ part,
                                                           int8_t* __restrict__ q, float* __restrict__ qs,
                                                           int* __restrict__ qsum) {
    constexpr int EPT = TT * EW / NT / TPT;                      // chains per thread: TPT x EPT
    constexpr int EG = EW / EPT;                                 // expert groups (threads per token group)
    constexpr int RS = router_stride<KS>(), K4 = KS / 4;
    constexpr int XV = TT * K4 / NT, WV = KS * (EW / 4) / NT;
    static_assert(XV * NT == TT * K4 && WV * NT == KS * (EW / 4) && TPT * EPT * NT == TT * EW && RKW % KS == 0 &&
                  KS % 128 == 0, "router tile");
    extern __shared__ __align__(16) float rl[];
    float* xs = rl;                       // [TT][RS]
    float* ws = rl + TT * RS;             // [EW][RS]: Wr slice transposed, k contiguous per expert
    // XCD-aware: workgroups go round-robin over the 8 XCDs by linear workgroup id.
    // - Above 32 tokens, K chunk c = id % 8 puts every workgroup of chunk c on XCD c: the chunk's Wr rows and x
    //   columns are fetched into that XCD's L2 only (512 tokens: 19.1 -> 17.9 us per router stage).
    // - At decode (8 experts per slice), slice (id % 8) X/8 + (id / 8) % (X/8) puts the 4 slices of a 128-byte Wr
    //   row segment on one XCD (config 1: 0.0545 -> 0.0539 ms per step; chunk per XCD: 0.0540 ms).
    static_assert(ROUTER_KC == 8, "one K chunk per XCD");
    const int X = gridDim.x;
    const int id = blockIdx.x + X * (blockIdx.y + gridDim.y * blockIdx.z);
    int c, sl, ty;
    if (EW == 8 && X % 8 == 0) {
        sl = (id % 8) * (X / 8) + (id / 8) % (X / 8);
        const int r = id / X;
        c = r % ROUTER_KC;
        ty = r / ROUTER_KC;
    } else {
        c = id % ROUTER_KC;
        sl = (id / ROUTER_KC) % X;
        ty = id / ROUTER_KC / X;
    }
    const int e0 = sl * EW, t0 = ty * TT;
    const int tid = threadIdx.x;
    // thread (token group tg, expert group eg): tokens tg TPT + i, experts j EG + eg (consecutive rows of the Wr
    // slice across a wave's lanes: conflict-free), one fma chain each over the chunk's k ascending
    const int tg = tid / EG, eg = tid % EG;
    float acc[TPT][EPT];
#pragma unroll
    for (int i = 0; i < TPT; ++i)
#pragma unroll
        for (int j = 0; j < EPT; ++j) acc[i][j] = 0.0f;
    for (int h = 0; h < RKW / KS; ++h) {
        const int kb = c * RKW + h * KS;
        float4 xv[XV], wv[WV];
#pragma unroll
        for (int i = 0; i < XV; ++i) {                            // x: TT x KS floats as float4
            const int idx = tid + NT * i, t = idx / K4, k4 = idx % K4;
            xv[i] = t0 + t < T ? *reinterpret_cast<const float4*>(x + size_t(t0 + t) * H + kb + 4 * k4)
                               : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        }
#pragma unroll
        for (int i = 0; i < WV; ++i) {                            // Wr: KS x EW floats as float4
            const int idx = tid + NT * i, k = idx / (EW / 4), e4 = idx % (EW / 4);
            wv[i] = *reinterpret_cast<const float4*>(Wr + size_t(kb + k) * E + e0 + 4 * e4);
        }
        if (h > 0) __syncthreads();                               // the previous sub-chunk has been read
#pragma unroll
        for (int i = 0; i < XV; ++i) {
            const int idx = tid + NT * i, t = idx / K4, k4 = idx % K4;
            *reinterpret_cast<float4*>(xs + t * RS + 4 * k4) = xv[i];
        }
#pragma unroll
        for (int i = 0; i < WV; ++i) {
            const int idx = tid + NT * i, k = idx / (EW / 4), e4 = idx % (EW / 4);
            ws[(4 * e4 + 0) * RS + k] = wv[i].x;
            ws[(4 * e4 + 1) * RS + k] = wv[i].y;
            ws[(4 * e4 + 2) * RS + k] = wv[i].z;
            ws[(4 * e4 + 3) * RS + k] = wv[i].w;
        }
        __syncthreads();
#pragma unroll 4
        for (int k = 0; k < KS; k += 4) {
            float4 a[TPT], b[EPT];
#pragma unroll
            for (int i = 0; i < TPT; ++i) a[i] = *reinterpret_cast<const float4*>(xs + (tg * TPT + i) * RS + k);
#pragma unroll
            for (int j = 0; j < EPT; ++j) b[j] = *reinterpret_cast<const float4*>(ws + (j * EG + eg) * RS + k);
#pragma unroll
            for (int i = 0; i < TPT; ++i)
#pragma unroll
                for (int j = 0; j < EPT; ++j) {
                    acc[i][j] = __builtin_fmaf(a[i].x, b[j].x, acc[i][j]);
                    acc[i][j] = __builtin_fmaf(a[i].y, b[j].y, acc[i][j]);
                    acc[i][j] = __builtin_fmaf(a[i].z, b[j].z, acc[i][j]);
                    acc[i][j] = __builtin_fmaf(a[i].w, b[j].w, acc[i][j]);
                }
        }
        if (q != nullptr) {
            // A8 of the sub-chunk's x slice (KS / 128 groups per token): LPT = KS / 8 lanes per token, 8 values each,
            // 64 / LPT tokens per wave job; wave w of expert slice b takes jobs w E/EW + b + i NWV E/EW, so the jobs
            // are spread over the expert slices' workgroups
            constexpr int NWV = NT / 64, LPT = KS / 8, TPW = 64 / LPT;
            const int lane = tid & 63;
            for (int j = (tid >> 6) * X + sl; j < TT / TPW; j += NWV * X) {
                const int tt = TPW * j + lane / LPT, l = lane % LPT;
                const float4 a = *reinterpret_cast<const float4*>(xs + tt * RS + 8 * l);
                const float4 b = *reinterpret_cast<const float4*>(xs + tt * RS + 8 * l + 4);
                const float v[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
                const int t = t0 + tt;   // (rows beyond T: computed on zeros, not written)
                const size_t gi = size_t(t) * (H / GROUP) + kb / GROUP + (l >> 4);
                quant_a8_8(v, lane, q + size_t(t) * H + kb + 8 * l, qs + gi, qsum + gi, t < T);
            }
        }
    }
#pragma unroll
    for (int i = 0; i < TPT; ++i) {
        const int t = t0 + tg * TPT + i;
        if (t < T)
#pragma unroll
            for (int j = 0; j < EPT; ++j) part[(size_t(c) * T + t) * E + e0 + j * EG + eg] = acc[i][j];
    }
}

// Selection keys: (value desc, index asc) as one unsigned 64-bit order: the float's bits mapped to an
// order-preserving unsigned integer in the high word, 0xFFFF - index in the low word; key 0 = no candidate.
__device__ __forceinline__ uint64_t sel_key(float v, int idx) {
    const uint32_t u = __float_as_uint(v);
    const uint32_t o = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
    return (uint64_t(o) << 32) | uint32_t(0xFFFF - idx);
}
__device__ __forceinline__ int key_index(uint64_t k) { return 0xFFFF - int(uint32_t(k) & 0xFFFFu); }




__device__ __forceinline__ uint64_t shfl_xor64(uint64_t v, int o) {
    const uint32_t lo = uint32_t(xor_lane(int(uint32_t(v)), o)), hi = uint32_t(xor_lane(int(uint32_t(v >> 32)), o));
    return (uint64_t(hi) << 32) | lo;
}

__device__ __forceinline__ int width_class(int bits) { return bits == 8 ? 0 : bits == 4 ? 1 : bits == 3 ? 2 : 3; }
// decode units, longest first: a streamed unit's time is set by its vector work, and the 2-bit units (4 strips per
// wave) have the most tiles (measured at 32 tokens against the byte order 8, 4, 3, 2 with the shared expert first:
// 0.0623 -> 0.0615 ms per step)

// the units of expert e: items of <= ntok of its c slots starting at slot st, each split into row blocks
__device__ void emit_units(int e, int c, int st, int ntok, int bits, int base_gu, int base_dn, Item* units_gu,
                           Item* units_dn) {
    const int nit = (c + ntok - 1) / ntok, rg = gemm_row_blocks(false, bits), rd = gemm_row_blocks(true, bits);
    for (int j = 0; j < nit; ++j) {
        const int s0 = st + j * ntok, n = min(ntok, c - j * ntok);
        for (int r = 0; r < rg; ++r) units_gu[base_gu + j * rg + r] = Item{e, s0, n, r};
        for (int r = 0; r < rd; ++r) units_dn[base_dn + j * rd + r] = Item{e, s0, n, r};
    }
}

// the shared expert's units (all T tokens, slots T K + t), the first of both lists; strided over the block
__device__ void emit_shared_units(int E, int T, int K, int ntok, int bits, Item* units_gu, Item* units_dn) {
    const int ns = (T + ntok - 1) / ntok, rg = gemm_row_blocks(false, bits), rd = gemm_row_blocks(true, bits);
    for (int u = threadIdx.x; u < ns * rg; u += blockDim.x) {
        const int j = u / rg;
        units_gu[u] = Item{E, T * K + j * ntok, min(ntok, T - j * ntok), u % rg};
    }
    for (int u = threadIdx.x; u < ns * rd; u += blockDim.x) {
        const int j = u / rd;
        units_dn[u] = Item{E, T * K + j * ntok, min(ntok, T - j * ntok), u % rd};
    }
}


// Cost of one row-block task of a chunk with nt 16-slot tiles, in 50 ns units: a per-row-block part (code
// unpacking, the weight stream) plus a per-tile part (MFMAs and the fp32 epilogue), as measured on MI355X for
// each code width (8-bit row blocks have half the rows)
__device__ __forceinline__ int rb_cost(int bits, int nt, bool down) {
    if (down) return bits == 8 ? 73 + 17 * nt : bits == 3 ? 37 + 18 * nt : bits == 4 ? 34 + 19 * nt : 30 + 18 * nt;
    return bits == 8 ? 64 + 35 * nt : bits == 3 ? 134 + 66 * nt : bits == 4 ? 78 + 72 * nt : 70 + 70 * nt;
}
// The activation staging a workgroup does for every chunk it touches (measured: ≈ 4.7 µs for gate_up, 64 slots x
// 2 KiB; ≈ 2.7 µs for down), costed at half weight at each chunk's start, so that workgroups that touch more
// chunks take fewer row blocks. (At full weight config 3 gained 2.6 % but 512-token layers, with under two row
// blocks per workgroup, lost 1.2 %; at half weight config 3 gains 1.8 %, config 4 1 %, and nothing loses.)
constexpr int STAGE_COST_GU = 48, STAGE_COST_DN = 28;
// the chunk's row-block task cost and row-block count of both GEMMs, packed (cost << 8 | count) for the planner
__device__ __forceinline__ void chunk_tasks(int bits, int ntok, uint32_t* gu, uint32_t* dn) {
    const int nt = (ntok + 15) >> 4;
    *gu = uint32_t(rb_cost(bits, nt, false) << 8) | uint32_t(tiled_row_blocks(false, bits));
    *dn = uint32_t(rb_cost(bits, nt, true) << 8) | uint32_t(tiled_row_blocks(true, bits));
}

// floor(x / d) for 0 <= x < 2^53, d > 0: a double quotient corrected by integer products
__device__ __forceinline__ long long floor_div(long long x, long long d) {
    long long q = (long long)(double(x) / double(d));
    while (q > 0 && q * d > x) --q;
    while ((q + 1) * d <= x) ++q;
    return q;
}



// Descending bitonic sort of one key per lane across the 64 lanes of a wave: lane i ends with the i-th largest.
__device__ __forceinline__ uint64_t wave_sort_desc(uint64_t k, int lane) {
#pragma unroll
    for (int s = 2; s <= 64; s <<= 1)
#pragma unroll
        for (int j = s >> 1; j > 0; j >>= 1) {
            const uint64_t o = shfl_xor64(k, j);
            // blocks of s lanes alternate direction (all descending at s = 64); the lower lane of a pair keeps
            // the larger key in a descending block
            const bool keep_max = ((lane & j) == 0) == ((lane & s) == 0);
            k = keep_max ? (o > k ? o : k) : (o < k ? o : k);
        }
    return k;
}



// ---- decode routing (one routing block, T <= block <= 32) ------------------------------------------------------
// score_kernel (with the pool), select_token_kernel (one token per workgroup), then dispatch_kernel (one
// workgroup: slots and work units for all tokens; or the gate_up GEMM of a layer forward, which plans for itself).
// DecodeState is zero when a call starts, and whichever kernel consumes it leaves it zero again.

// With qx.x set, the workgroup of token t first writes the A8 of x's row t (H = 2048: wave w takes columns
// 512 w .. 512 w + 511), so routing from given logits needs no launch of its own for it.
__device__ __forceinline__ void row_a8(const QuantX& qx, int t) {
    if (qx.x == nullptr) return;
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const size_t base = size_t(t) * 2048 + 512 * w, gi = size_t(t) * 16 + 4 * w;
    quant_a8_512(qx.x + base, lane, qx.q + base, qx.s + gi, qx.sum + gi);
}

// grid T, 256 threads (thread = expert): logit = partials summed in chunk order; sig[t, e] = sigmoid(logit);
// with the pool, blockmax[e] = max over tokens of the ordered key of sigmoid + bias
template <bool QA8>
__global__ void __launch_bounds__(256) score_kernel(const float* __restrict__ part, int nchunks,
                                                    const float* __restrict__ bias, int T, int E, int block,
                                                    int pool_on, float* __restrict__ sig,
                                                    uint32_t* __restrict__ blockmax, QuantX qx) {
    const int t = blockIdx.x, e = threadIdx.x;
    if constexpr (QA8) row_a8(qx, t);
    if (e >= E) return;
    float p[ROUTER_KC];
#pragma unroll
    for (int c = 0; c < ROUTER_KC; ++c) p[c] = c < nchunks ? part[(size_t(c) * T + t) * E + e] : 0.0f;
    float l = p[0];
#pragma unroll
    for (int c = 1; c < ROUTER_KC; ++c)
        if (c < nchunks) l = l + p[c];
    const float sg = sigmoid_f32(l);
    sig[size_t(t) * E + e] = sg;
    if (pool_on) atomicMax(&blockmax[size_t(t / block) * E + e], okey(sg + bias[e]));
}


// Slots and work units of the decode step (engine/ops.cu:333-370), one workgroup of 256 threads (thread e writes
// expert e's units); the masks and pool maxima are left zero for the next call.
__global__ void __launch_bounds__(256) dispatch_kernel(int T, int E, int K, const int* __restrict__ topk,
                                                       const float* __restrict__ topw, DecodeState ds, DispatchOut d) {
    __shared__ DecodePlan P;
    decode_plan_scan(E, ds.tmask, d.bits, P);
    const int e = threadIdx.x;
    if (e < E) {
        ds.tmask[e] = 0u;
        ds.blockmax[e] = 0u;
        decode_plan_write_expert(P, e, 0, 1, d);
    }
    decode_plan_write_rest(P, e, 256, T, E, K, topk, topw, d);
}


// Decode selection, one token per workgroup (engine/ops.cu:256-327): thread e scores expert e, each wave sorts
// its 64 keys, wave 0 sorts the four waves' leaders and writes the top-K, the routing weights
// (engine/ops.cu:298-321) and the token masks. Without the pool the scores come from the router partials (summed
// in chunk order, then the sigmoid); with it from score_kernel's sigmoids, and expert e is in the block's pool
// when fewer than C experts have a larger blockmax key (ties to the lower index): the four waves sort the
// blockmax keys and each thread counts the larger ones by binary search. One token per workgroup puts T times
// more waves on this latency-bound step than 8 tokens per workgroup.
template <bool POOL, bool QA8>
__global__ void __launch_bounds__(256) select_token_kernel(const float* __restrict__ part, int nchunks,
                                                           const float* __restrict__ sig,
                                                           const float* __restrict__ bias, int T, int E, int K,
                                                           int C, int block, float rscale, int* __restrict__ topk,
                                                           float* __restrict__ topw, DecodeState ds, QuantX qx) {
    __shared__ float sig_s[MAXE];
    __shared__ uint64_t lead[4 * 8];
    __shared__ uint64_t pool_s[POOL ? MAXE : 1];
    const int t = blockIdx.x, e = threadIdx.x, lane = e & 63, w = e >> 6;
    if constexpr (QA8) row_a8(qx, t);
    bool inpool = true;
    if constexpr (POOL) {
        const uint64_t pk =
            e < E ? (uint64_t(ds.blockmax[size_t(t / block) * E + e]) << 32) | uint32_t(0xFFFF - e) : 0ull;
        pool_s[w * 64 + lane] = wave_sort_desc(pk, lane);
        __syncthreads();
        int rank = 0;
#pragma unroll
        for (int v = 0; v < 4; ++v) {   // keys of the descending list v larger than pk
            const uint64_t* a = pool_s + v * 64;
            int lo = 0;
#pragma unroll
            for (int step = 32; step > 0; step >>= 1)
                if (a[lo + step - 1] > pk) lo += step;
            if (lo == 63 && a[63] > pk) lo = 64;
            rank += lo;
        }
        inpool = rank < C;
    }
    uint64_t key = 0ull;
    if (e < E) {
        float sv;
        if constexpr (POOL) {
            sv = sig[size_t(t) * E + e];
        } else {
            float p[ROUTER_KC];
#pragma unroll
            for (int c = 0; c < ROUTER_KC; ++c) p[c] = c < nchunks ? part[(size_t(c) * T + t) * E + e] : 0.0f;
            float l = p[0];
#pragma unroll
            for (int c = 1; c < ROUTER_KC; ++c)
                if (c < nchunks) l = l + p[c];
            sv = sigmoid_f32(l);
        }
        sig_s[e] = sv;
        if (inpool) key = sel_key(sv + bias[e], e);
    }
    key = wave_sort_desc(key, lane);
    if (lane < 8) lead[w * 8 + lane] = key;
    __syncthreads();
    if (w == 0) {
        uint64_t k2 = lane < 32 ? lead[lane] : 0ull;
        k2 = wave_sort_desc(k2, lane);
        const int ex = key_index(k2);
        const float sk = lane < K ? sig_s[ex] : 0.0f;
        float wsum = 0.0f;
#pragma unroll
        for (int k = 0; k < 8; ++k)
            if (k < K) wsum = wsum + __int_as_float(__builtin_amdgcn_readlane(__float_as_int(sk), k));
        if (lane < K) {
            topk[size_t(t) * K + lane] = ex;
            topw[size_t(t) * K + lane] = sk / (wsum + 1e-20f) * rscale;
            atomicOr(&ds.tmask[size_t(t / block) * E + ex], 1u << (t % block));
        }
    }
}


// Token masks of externally given routing. grid nb, 256 threads.
__global__ void __launch_bounds__(256) masks_kernel(const int* __restrict__ topk, int T, int E, int K, int block,
                                                    uint32_t* __restrict__ mask) {
    __shared__ uint32_t tmask[MAXE];
    const int b = blockIdx.x, t0 = b * block, tb = min(block, T - t0);
    if (threadIdx.x < E) tmask[threadIdx.x] = 0u;
    __syncthreads();
    for (int p = threadIdx.x; p < tb * K; p += blockDim.x) {
        const int t = p / K, k = p % K;
        atomicOr(&tmask[topk[size_t(t0 + t) * K + k]], 1u << t);
    }
    __syncthreads();
    if (threadIdx.x < E) mask[size_t(b) * E + threadIdx.x] = tmask[threadIdx.x];
}

// Slot ranges and work units (engine/ops.cu:333-370, :384-410): slots expert-major (expert ascending), inside
// an expert block-major then token-ascending. An expert with more than TILED_MIN slots (when `tiled`) gets tiled
// units (chunks of <= TILED_NTOK slots x tiled row blocks), otherwise streamed units (items of <= ntok slots x
// streamed row blocks). Both lists are ordered heaviest first (shared expert, then 8 / 4 / 3 / 2-bit experts).
// One workgroup of four threads per expert: the block masks are split in four contiguous ranges.
__global__ void __launch_bounds__(PLAN_NT) plan_kernel(const uint32_t* __restrict__ mask, int T, int E, int K,
                                                       int block, int has_shared, int ntok, int tiled,
                                                       const int8_t* __restrict__ bits, int* __restrict__ count,
                                                       int* __restrict__ start, int* __restrict__ bpre,
                                                       Item* __restrict__ units_gu, Item* __restrict__ units_dn,
                                                       Item* __restrict__ tunits_gu, Item* __restrict__ tunits_dn,
                                                       int* __restrict__ n_units, int g_gu, int g_dn,
                                                       int* __restrict__ tstart, int max_chunks) {
    constexpr int NP = PLAN_NT / MAXE;         // threads per expert: each takes a contiguous range of blocks
    constexpr int NBR = MAXB_BLOCKS / NP;      // block masks of a range held in registers
    constexpr int NWAVE = PLAN_NT / 64;
    // chunk tables (max_chunks entries): row-block tasks of both GEMMs, then their positions [n_chunks + 1]
    extern __shared__ uint32_t plan_lds[];
    uint32_t* task_gu = plan_lds;
    uint32_t* task_dn = task_gu + max_chunks;
    int* pre_gu = reinterpret_cast<int*>(task_dn + max_chunks);
    int* pre_dn = pre_gu + max_chunks + 1;
    int* owner = pre_dn + max_chunks + 1;      // expert of each chunk
    __shared__ int wt_i[NWAVE], wt_c[NWAVE];
    __shared__ uint64_t wt[4][4];
    __shared__ uint64_t tot[4];
    __shared__ int first_l[MAXE + 1], cnt_l[MAXE + 1], st_l[MAXE + 1], bits_l[MAXE + 1];
    __shared__ int cpart_s[NP][MAXE];          // tokens of expert e in part p's block range
    const int tid = threadIdx.x, e = tid % MAXE, part = tid / MAXE, nb = (T + block - 1) / block;
    const int lane = tid & 63, wv = tid >> 6, w = wv & 3;   // (w: the wave within the expert-scan group)
    const bool g0 = part == 0;                 // the expert's lead thread (scans, units)
    // token masks of the part's block range [b_lo, b_hi): unconditional loads at clamped indices, so that the
    // batch is issued back to back
    const int ec = min(e, E - 1), nbp = (nb + NP - 1) / NP, b_lo = min(nb, part * nbp), b_hi = min(nb, b_lo + nbp);
    // code widths read up front, with the masks: a load after them would expose its own latency
    const int bw_ld = bits[ec], sbits_ld = has_shared ? bits[E] : 8;
    uint32_t mv[NBR];
#pragma unroll
    for (int j = 0; j < NBR; ++j) mv[j] = mask[size_t(min(b_lo + j, nb - 1)) * E + ec];
    int cp = 0;
#pragma unroll
    for (int j = 0; j < NBR; ++j) cp += b_lo + j < b_hi ? __popc(mv[j]) : 0;
    for (int b0 = b_lo + NBR; b0 < b_hi; b0 += 16) {   // ranges longer than the registers hold
        uint32_t m2[16];
#pragma unroll
        for (int j = 0; j < 16; ++j) m2[j] = mask[size_t(min(b0 + j, nb - 1)) * E + ec];
#pragma unroll
        for (int j = 0; j < 16; ++j) cp += b0 + j < b_hi ? __popc(m2[j]) : 0;
    }
    if (e >= E) cp = 0;
    cpart_s[part][e] = cp;
    __syncthreads();
    int c = 0, cbefore = 0;   // the expert's slots; those in the blocks before the part's range
#pragma unroll
    for (int pp = 0; pp < NP; ++pp) {
        const int v = cpart_s[pp][e];
        cbefore += pp < part ? v : 0;
        c += v;
    }
    const bool big = e < E && tiled && c > 0;
    const bool sbig = has_shared && tiled;
    const int nsch = sbig ? tiled_chunks(T) : 0;
    const int bw = e < E ? bw_ld : 2, cls = width_class(bw);
    const int nit = e < E && !big ? (c + ntok - 1) / ntok : 0, nch = big ? tiled_chunks(c) : 0;
    // one pass of inclusive scans over the experts (lead threads): slots, tiled chunks, and per width class
    // (16-bit fields) the streamed units of both lists and the tiled chunks
    int incl = c;
    uint64_t s0 = uint64_t(nit * gemm_row_blocks(false, bw)) << (16 * cls);
    uint64_t s1 = uint64_t(nit * gemm_row_blocks(true, bw)) << (16 * cls);
    uint64_t t0 = uint64_t(nch) << (16 * cls);
    const uint64_t own0 = s0, own1 = s1, ownt = t0;
    incl = wave_incl_scan(incl);
    s0 = wave_incl_scan(s0);
    s1 = wave_incl_scan(s1);
    t0 = wave_incl_scan(t0);
    if (g0 && lane == 63) {
        wt_i[w] = incl;
        wt[w][0] = s0;
        wt[w][1] = s1;
        wt[w][2] = t0;
    }
    __syncthreads();
    for (int i = 0; i < w; ++i) {
        incl += wt_i[i];
        s0 += wt[i][0];
        s1 += wt[i][1];
        t0 += wt[i][2];
    }
    if (tid == MAXE - 1) {
        tot[0] = s0;
        tot[1] = s1;
        tot[2] = t0;
    }
    __syncthreads();
    const int sbits = sbits_ld;
    const int ns = has_shared && !sbig ? (T + ntok - 1) / ntok : 0;
    // offsets: the shared expert's units first, then width classes 0 .. 3 (8, 4, 3, 2 bits), expert ascending
    int bg = ns * gemm_row_blocks(false, sbits), bd = ns * gemm_row_blocks(true, sbits), bt = nsch;
    int og = 0, od = 0, ot = 0;
    for (int k = 0; k < 4; ++k) {
        if (k == cls) {
            og = bg + int(((s0 - own0) >> (16 * k)) & 0xFFFFu);
            od = bd + int(((s1 - own1) >> (16 * k)) & 0xFFFFu);
            ot = bt + int(((t0 - ownt) >> (16 * k)) & 0xFFFFu);
        }
        bg += int((tot[0] >> (16 * k)) & 0xFFFFu);
        bd += int((tot[1] >> (16 * k)) & 0xFFFFu);
        bt += int((tot[2] >> (16 * k)) & 0xFFFFu);
    }
    // (the scans above ran in every part on identical values; only part 0's results are used below)
    const int st = incl - c;
    if (e < E) {
        // slot base of each (block, expert) of the part's range
        int run = st + cbefore;
#pragma unroll
        for (int j = 0; j < NBR; ++j)
            if (b_lo + j < b_hi) {
                bpre[size_t(b_lo + j) * E + e] = run;
                run += __popc(mv[j]);
            }
        for (int b0 = b_lo + NBR; b0 < b_hi; b0 += 16) {
            uint32_t m2[16];
#pragma unroll
            for (int j = 0; j < 16; ++j) m2[j] = mask[size_t(min(b0 + j, nb - 1)) * E + e];
#pragma unroll
            for (int j = 0; j < 16; ++j)
                if (b0 + j < b_hi) {
                    bpre[size_t(b0 + j) * E + e] = run;
                    run += __popc(m2[j]);
                }
        }
    }
    if (g0 && e < E) {
        count[e] = c;
        start[e] = st;
        if (big) {   // the chunks are written below, one thread per chunk
            first_l[e] = ot;
            cnt_l[e] = c;
            st_l[e] = st;
            bits_l[e] = bw;
            for (int j = 0; j < nch; ++j) owner[ot + j] = e;
        } else {
            emit_units(e, c, st, ntok, bw, og, od, units_gu, units_dn);
        }
    }
    if (ns) emit_shared_units(E, T, K, ntok, sbits, units_gu, units_dn);
    if (sbig) {
        if (tid == 0) {
            first_l[E] = 0;
            cnt_l[E] = T;
            st_l[E] = T * K;
            bits_l[E] = sbits;
        }
        for (int j = tid; j < nsch; j += blockDim.x) owner[j] = E;
    }
    if (tid == 0) {
        n_units[0] = bg;
        n_units[1] = bd;
        n_units[2] = bt;
        n_units[3] = bt;
    }
    if (!tiled) return;
    // the tiled chunks: tiled_per(c) slots of an expert's c each, the last one shorter (Item.rb unused)
    __syncthreads();
    const int n = bt;
    for (int j = tid; j < n; j += blockDim.x) {
        const int x = owner[j], cx = cnt_l[x], pc = tiled_per(cx), jj = j - first_l[x];
        const Item it{x, st_l[x] + jj * pc, min(pc, cx - jj * pc), 0};
        tunits_gu[j] = it;
        tunits_dn[j] = it;
        chunk_tasks(bits_l[x], it.ntok, &task_gu[j], &task_dn[j]);
    }
    // chunk positions of both GEMMs: scans of the chunk costs (each thread a run of consecutive chunks)
    __syncthreads();
    const int per = (n + blockDim.x - 1) / blockDim.x, j0 = min(n, tid * per), j1 = min(n, j0 + per);
    auto cost = [](uint32_t t, int stage) { return stage + int(t >> 8) * int(t & 255u); };
    int run0 = 0, run1 = 0;
    for (int j = j0; j < j1; ++j) {
        run0 += cost(task_gu[j], STAGE_COST_GU);
        run1 += cost(task_dn[j], STAGE_COST_DN);
    }
    int inc0 = run0, inc1 = run1;
    inc0 = wave_incl_scan(inc0);
    inc1 = wave_incl_scan(inc1);
    if (lane == 63) {
        wt_i[wv] = inc0;
        wt_c[wv] = inc1;
    }
    __syncthreads();
    for (int i = 0; i < wv; ++i) {
        inc0 += wt_i[i];
        inc1 += wt_c[i];
    }
    run0 = inc0 - run0;
    run1 = inc1 - run1;
    for (int j = j0; j < j1; ++j) {
        pre_gu[j] = run0;
        pre_dn[j] = run1;
        run0 += cost(task_gu[j], STAGE_COST_GU);
        run1 += cost(task_dn[j], STAGE_COST_DN);
    }
    if (tid == int(blockDim.x) - 1) {
        pre_gu[n] = inc0;
        pre_dn[n] = inc1;
    }
    __syncthreads();
    // work partition: workgroup q starts at task position lo_q = ceil(q C / G); the chunk j holding it
    // (pre[j] <= lo_q < pre[j + 1]) is found by binary search, and the task inside it is the first row block
    // whose cost span (after the chunk's staging cost) starts at or after lo_q (one past the chunk's last: the
    // next chunk's first)
    // (both GEMMs' partitions at once: thread i takes workgroup i of gate_up, or i - g_gu of down)
    if (tid == 0) {
        tstart[g_gu] = n;
        tstart[g_gu + 1 + g_dn] = n;
    }
    for (int idx = tid; idx < g_gu + g_dn; idx += blockDim.x) {
        const int m = idx >= g_gu, q = m ? idx - g_gu : idx;
        const int G = m ? g_dn : g_gu;
        const int* P = m ? pre_dn : pre_gu;
        const uint32_t* task = m ? task_dn : task_gu;
        int* ts = tstart + (m ? g_gu + 1 : 0);
        const long long C = P[n];
        const long long lo = C == 0 ? 0 : floor_div((long long)q * C + G - 1, G);
        if (lo >= C) {
            ts[q] = n;
            continue;
        }
        int a = 0, b = n;   // P[a] <= lo < P[b]
        while (b - a > 1) {
            const int mid = (a + b) >> 1;
            if (P[mid] <= lo) a = mid;
            else b = mid;
        }
        const int nrb = int(task[a] & 255u), span = int(task[a] >> 8);
        const long long off = lo - P[a] - (m ? STAGE_COST_DN : STAGE_COST_GU);
        const int r = off <= 0 ? 0 : int((off + span - 1) / span);
        ts[q] = r >= nrb ? a + 1 : (a | (r << TASK_RB_SHIFT));
    }
}

// Place every (token, k) pair in its slot; tok_slots[t, K] = the shared slot (or -1). grid nb, 256 threads.
__global__ void __launch_bounds__(256) place_kernel(const int* __restrict__ topk, const float* __restrict__ topw,
                                                    uint32_t* __restrict__ mask, uint32_t* __restrict__ blockmax,
                                                    const int* __restrict__ bpre, int T, int E, int K, int block,
                                                    int has_shared,
                                                    int* __restrict__ slot_token, float* __restrict__ slot_weight,
                                                    int* __restrict__ tok_slots) {
    // the block's masks and slot bases staged in LDS while the (token, k) pairs load, so the slot of a pair
    // costs one global round trip
    __shared__ uint32_t m_s[MAXE];
    __shared__ int bp_s[MAXE];
    const int b = blockIdx.x, t0 = b * block, tb = min(block, T - t0);
    for (int e = threadIdx.x; e < E; e += blockDim.x) {
        m_s[e] = mask[size_t(b) * E + e];
        bp_s[e] = bpre[size_t(b) * E + e];
    }
    __syncthreads();
    for (int p = threadIdx.x; p < tb * K; p += blockDim.x) {
        const int tl = p / K, k = p % K, t = t0 + tl;
        const int ex = topk[size_t(t) * K + k];
        const int sl = bp_s[ex] + __popc(m_s[ex] & ((1u << tl) - 1u));
        slot_token[sl] = t;
        slot_weight[sl] = topw[size_t(t) * K + k];
        tok_slots[size_t(t) * (K + 1) + k] = sl;
    }
    for (int tl = threadIdx.x; tl < tb; tl += blockDim.x) {
        const int t = t0 + tl;
        if (has_shared) {
            slot_token[T * K + t] = t;
            slot_weight[T * K + t] = 1.0f;
        }
        tok_slots[size_t(t) * (K + 1) + K] = has_shared ? T * K + t : -1;
    }
    // the block's token masks and pool maxima are consumed: leave them zero for the next call's atomics
    __syncthreads();
    for (int e = threadIdx.x; e < E; e += blockDim.x) {
        mask[size_t(b) * E + e] = 0u;
        blockmax[size_t(b) * E + e] = 0u;
    }
}

}  // namespace

hipError_t launch_router_logits(const float* x, const float* Wr, int T, int H, int E, float* part, int8_t* q,
                                float* qs, int* qsum, hipStream_t st) {
    static bool attr = false;
    if (!attr) {
        hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(router_logits_kernel<32, 8, 256, 1, 256>),
                                           hipFuncAttributeMaxDynamicSharedMemorySize, router_lds<32, 8, 256>());
        if (e == hipSuccess)
            e = hipFuncSetAttribute(reinterpret_cast<const void*>(router_logits_kernel<64, 64, 512, 2, 128>),
                                    hipFuncAttributeMaxDynamicSharedMemorySize, router_lds<64, 64, 128>());
        if (e != hipSuccess) return e;
        attr = true;
    }
    if (T <= 32) {
        const dim3 grid(E / 8, 1, ROUTER_KC);
        router_logits_kernel<32, 8, 256, 1, 256><<<grid, 256, router_lds<32, 8, 256>(), st>>>(x, Wr, T, H, E, part, q,
                                                                                             qs, qsum);
    } else {
        const dim3 grid(E / 64, (T + 63) / 64, ROUTER_KC);
        router_logits_kernel<64, 64, 512, 2, 128><<<grid, 512, router_lds<64, 64, 128>(), st>>>(x, Wr, T, H, E, part,
                                                                                                q, qs, qsum);
    }
    return hipGetLastError();
}

hipError_t launch_route(const float* part, int nchunks, const float* bias, int T, int E, int K, int C, int block,
                        float rscale, float* sig, uint32_t* blockmax, int32_t* topk, float* topw, uint32_t* mask,
                        const QuantX& qx, hipStream_t st) {
    if (E > MAXE || block > MAXB) return hipErrorInvalidValue;
    const DecodeState ds{blockmax, mask};
    if (C < E) {
        if (qx.x) score_kernel<true><<<T, 256, 0, st>>>(part, nchunks, bias, T, E, block, 1, sig, blockmax, qx);
        else score_kernel<false><<<T, 256, 0, st>>>(part, nchunks, bias, T, E, block, 1, sig, blockmax, qx);
        select_token_kernel<true, false><<<T, 256, 0, st>>>(part, nchunks, sig, bias, T, E, K, C, block, rscale,
                                                             topk, topw, ds, QuantX{});
    } else if (qx.x) {
        select_token_kernel<false, true><<<T, 256, 0, st>>>(part, nchunks, sig, bias, T, E, K, C, block, rscale,
                                                             topk, topw, ds, qx);
    } else {
        select_token_kernel<false, false><<<T, 256, 0, st>>>(part, nchunks, sig, bias, T, E, K, C, block, rscale,
                                                              topk, topw, ds, qx);
    }
    return hipGetLastError();
}

hipError_t launch_decode_route(const float* part, int nchunks, const float* bias, int T, int E, int K, int C,
                               float rscale, float* sig, int32_t* topk, float* topw, uint32_t* blockmax,
                               uint32_t* tmask, int has_shared, const int8_t* bits, int32_t* count, int32_t* start,
                               Item* units_gu, Item* units_dn, int* n_units, int32_t* slot_token, float* slot_weight,
                               int32_t* tok_slots, const QuantX& qx, int dispatch, hipStream_t st) {
    if (T > 32 || E > MAXE) return hipErrorInvalidValue;
    const DecodeState ds{blockmax, tmask};
    if (C < E) {
        if (qx.x) score_kernel<true><<<T, 256, 0, st>>>(part, nchunks, bias, T, E, MAXB, 1, sig, blockmax, qx);
        else score_kernel<false><<<T, 256, 0, st>>>(part, nchunks, bias, T, E, MAXB, 1, sig, blockmax, qx);
        select_token_kernel<true, false><<<T, 256, 0, st>>>(part, nchunks, sig, bias, T, E, K, C, MAXB, rscale, topk,
                                                             topw, ds, QuantX{});
    } else if (qx.x) {
        select_token_kernel<false, true><<<T, 256, 0, st>>>(part, nchunks, sig, bias, T, E, K, C, MAXB, rscale, topk,
                                                             topw, ds, qx);
    } else {
        select_token_kernel<false, false><<<T, 256, 0, st>>>(part, nchunks, sig, bias, T, E, K, C, MAXB, rscale,
                                                              topk, topw, ds, qx);
    }
    const DispatchOut d{has_shared, 16, bits, count, start, units_gu, units_dn, n_units, slot_token, slot_weight,
                        tok_slots};
    if (dispatch) dispatch_kernel<<<1, 256, 0, st>>>(T, E, K, topk, topw, ds, d);
    return hipGetLastError();
}

__global__ void __launch_bounds__(256) zero_u32_kernel(uint32_t* __restrict__ a, uint32_t* __restrict__ b, int n) {
    for (int i = threadIdx.x; i < n; i += blockDim.x) {
        a[i] = 0u;
        b[i] = 0u;
    }
}

hipError_t launch_zero_decode_state(uint32_t* blockmax, uint32_t* tmask, int E, hipStream_t st) {
    zero_u32_kernel<<<1, 256, 0, st>>>(blockmax, tmask, E);
    return hipGetLastError();
}

hipError_t launch_masks(const int32_t* topk, int T, int E, int K, int block, uint32_t* mask, hipStream_t st) {
    const int nb = (T + block - 1) / block;
    masks_kernel<<<nb, 256, 0, st>>>(topk, T, E, K, block, mask);
    return hipGetLastError();
}

hipError_t launch_plan(const uint32_t* mask, int T, int E, int K, int block, int has_shared, int ntok, int tiled,
                       const int8_t* bits, int32_t* count, int32_t* start, int32_t* bpre, Item* units_gu,
                       Item* units_dn, Item* tunits_gu, Item* tunits_dn, int* n_units, int g_gu, int g_dn,
                       int* tstart, int max_chunks, hipStream_t st) {
    const size_t lds = (5 * size_t(max_chunks) + 2) * sizeof(uint32_t);
    plan_kernel<<<1, PLAN_NT, lds, st>>>(mask, T, E, K, block, has_shared, ntok, tiled, bits, count, start, bpre,
                                     units_gu, units_dn, tunits_gu, tunits_dn, n_units, g_gu, g_dn, tstart,
                                     max_chunks);
    return hipGetLastError();
}

hipError_t launch_place(const int32_t* topk, const float* topw, uint32_t* mask, uint32_t* blockmax,
                        const int32_t* bpre, int T, int E, int K, int block, int has_shared, int32_t* slot_token,
                        float* slot_weight, int32_t* tok_slots, hipStream_t st) {
    const int nb = (T + block - 1) / block;
    place_kernel<<<nb, 256, 0, st>>>(topk, topw, mask, blockmax, bpre, T, E, K, block, has_shared, slot_token,
                                     slot_weight, tok_slots);
    return hipGetLastError();
}

}  // namespace llmoe
