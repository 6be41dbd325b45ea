// Router and dispatch kernels (engine/ops.cu:137-423): router logits, per-block sigmoid+bias scoring with the
// block expert pool and per-token top-K, routing weights, and the deterministic counting sort of (token, k)
// pairs into expert-major slots with the GEMM work items. All counts stay on the device.
#include "llmoe_internal.h"

namespace llmoe {

namespace {

constexpr int MAXB = 32;    // tokens per routing block (one 32-bit token mask per expert)
constexpr int MAXE = 256;   // experts (one thread each)

// logits partial c: fma chain over k = c H/8 .. (c+1) H/8 - 1 ascending from 0 (the summation order is fixed so
// the CPU checker reproduces it). Workgroup tile: 32 tokens x 64 experts of one K chunk, the chunk's x and Wr
// slices staged in LDS by one batch of loads; thread: 2 tokens x 4 experts.
// grid (E/64, ceil(T/32), 8), 256 threads, dynamic LDS ROUTER_LDS.
constexpr int RKW = 256;                                          // K per chunk (H = 2048)
constexpr int ROUTER_LDS = (32 * (RKW + 4) + RKW * 64) * 4;
__global__ void __launch_bounds__(256) router_logits_kernel(const float* __restrict__ x, const float* __restrict__ Wr,
                                                            int T, int H, int E, float* __restrict__ part) {
    extern __shared__ __align__(16) float rl[];
    float* xs = rl;                       // [32][RKW + 4]
    float* ws = rl + 32 * (RKW + 4);      // [RKW][64]
    const int e0 = blockIdx.x * 64, t0 = blockIdx.y * 32, c = blockIdx.z, kb = c * RKW;
    const int tid = threadIdx.x, ty = tid >> 4, tx = tid & 15;
#pragma unroll
    for (int i = 0; i < 8; ++i) {                                 // x: 32 x 256 floats as float4
        const int idx = tid + 256 * i, t = idx >> 6, k4 = idx & 63;
        const float4 v = t0 + t < T ? *reinterpret_cast<const float4*>(x + size_t(t0 + t) * H + kb + 4 * k4)
                                    : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        *reinterpret_cast<float4*>(xs + t * (RKW + 4) + 4 * k4) = v;
    }
#pragma unroll
    for (int i = 0; i < 16; ++i) {                                // Wr: 256 x 64 floats as float4
        const int idx = tid + 256 * i, k = idx >> 4, e4 = idx & 15;
        *reinterpret_cast<float4*>(ws + k * 64 + 4 * e4) =
            *reinterpret_cast<const float4*>(Wr + size_t(kb + k) * E + e0 + 4 * e4);
    }
    __syncthreads();
    float acc[2][4] = {{0.0f, 0.0f, 0.0f, 0.0f}, {0.0f, 0.0f, 0.0f, 0.0f}};
    const float* xa = xs + (2 * ty) * (RKW + 4);
    const float* xb = xa + (RKW + 4);
#pragma unroll 8
    for (int k = 0; k < RKW; ++k) {
        const float a = xa[k], b = xb[k];
        const float4 w = *reinterpret_cast<const float4*>(ws + k * 64 + 4 * tx);
        const float wv[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            acc[0][j] = __builtin_fmaf(a, wv[j], acc[0][j]);
            acc[1][j] = __builtin_fmaf(b, wv[j], acc[1][j]);
        }
    }
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const int t = t0 + 2 * ty + i;
        if (t < T)
            *reinterpret_cast<float4*>(part + (size_t(c) * T + t) * E + e0 + 4 * tx) =
                make_float4(acc[i][0], acc[i][1], acc[i][2], acc[i][3]);
    }
}

__device__ __forceinline__ bool beats(float a, int ia, float b, int ib) { return a > b || (a == b && ia < ib); }

// Selection keys: (value desc, index asc) as one unsigned 64-bit order: the float's bits mapped to an
// order-preserving unsigned integer in the high word, 0xFFFF - index in the low word; key 0 = no candidate.
__device__ __forceinline__ uint64_t sel_key(float v, int idx) {
    const uint32_t u = __float_as_uint(v);
    const uint32_t o = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
    return (uint64_t(o) << 32) | uint32_t(0xFFFF - idx);
}
__device__ __forceinline__ int key_index(uint64_t k) { return 0xFFFF - int(uint32_t(k) & 0xFFFFu); }

__device__ __forceinline__ void cas(uint64_t (&k)[8], int i, int l) {   // afterwards k[i] >= k[l]
    const uint64_t a = k[i], b = k[l];
    const bool sw = b > a;
    k[i] = sw ? b : a;
    k[l] = sw ? a : b;
}

// bitonic sorting network on 8 keys, largest first
__device__ __forceinline__ void sort8(uint64_t (&k)[8]) {
#pragma unroll
    for (int s = 2; s <= 8; s <<= 1)
#pragma unroll
        for (int j = s >> 1; j > 0; j >>= 1)
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const int l = i ^ j;
                if (l > i) {
                    if ((i & s) == 0) cas(k, i, l);
                    else cas(k, l, i);
                }
            }
}

// k <- largest 8 of two largest-first sorted lists: max(k[i], w[7 - i]) is bitonic and holds them; a 3-stage
// bitonic merge sorts it
__device__ __forceinline__ void merge8(uint64_t (&k)[8], const uint64_t (&w)[8]) {
#pragma unroll
    for (int i = 0; i < 8; ++i) k[i] = w[7 - i] > k[i] ? w[7 - i] : k[i];
#pragma unroll
    for (int j = 4; j > 0; j >>= 1)
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const int l = i ^ j;
            if (l > i) cas(k, i, l);
        }
}

__device__ __forceinline__ uint64_t shfl_xor64(uint64_t v, int o) {
    const uint32_t lo = __shfl_xor(uint32_t(v), o), hi = __shfl_xor(uint32_t(v >> 32), o);
    return (uint64_t(hi) << 32) | lo;
}

// exclusive prefix sums of two per-expert values over E <= 256 experts, by wave 0 (4 experts per lane);
// results in LDS arrays ex_a/ex_b, totals in tot[0..1]. All threads must call it (it synchronises).
__device__ void expert_scan2(const int* va, const int* vb, int E, int* ex_a, int* ex_b, int* tot) {
    if (threadIdx.x < 64) {
        const int l = threadIdx.x;
        int a[4], b[4], sa = 0, sb = 0;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int e = 4 * l + j;
            a[j] = e < E ? va[e] : 0;
            b[j] = e < E ? vb[e] : 0;
            sa += a[j];
            sb += b[j];
        }
        int ia = sa, ib = sb;   // inclusive scan over lanes
#pragma unroll
        for (int o = 1; o < 64; o <<= 1) {
            const int ta = __shfl_up(ia, o), tb2 = __shfl_up(ib, o);
            if (l >= o) {
                ia += ta;
                ib += tb2;
            }
        }
        int ra = ia - sa, rb = ib - sb;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int e = 4 * l + j;
            if (e < E) {
                ex_a[e] = ra;
                ex_b[e] = rb;
            }
            ra += a[j];
            rb += b[j];
        }
        if (l == 63) {
            tot[0] = ia;
            tot[1] = ib;
        }
    }
    __syncthreads();
}

// exclusive prefix sum over the NT threads of a block (Hillis-Steele in LDS); *total = the full sum
template <int NT>
__device__ int block_excl_scan(int v, int* buf, int* total) {
    const int i = threadIdx.x;
    buf[i] = v;
    __syncthreads();
    for (int o = 1; o < NT; o <<= 1) {
        const int add = i >= o ? buf[i - o] : 0;
        __syncthreads();
        buf[i] += add;
        __syncthreads();
    }
    const int incl = buf[i];
    *total = buf[NT - 1];
    __syncthreads();
    return incl - v;
}

// Work-unit offsets ordered heaviest first: the shared expert's units, then routed experts by code width (8, 4,
// 3, 2 bits), expert ascending inside a width -- long workgroups start first. Wave 0, 4 experts per lane.
// nu_gu / nu_dn: units per expert (LDS); cls: width class 0..3 per expert (LDS); sh_gu / sh_dn: shared units.
// Out (LDS): base_gu / base_dn per expert, tot[0] / tot[1] = total units. All threads must call it.
__device__ void unit_offsets(const int* nu_gu, const int* nu_dn, const int* cls, int E, int sh_gu, int sh_dn,
                             int* base_gu, int* base_dn, int* tot) {
    if (threadIdx.x < 64) {
        const int l = threadIdx.x;
        int bg = sh_gu, bd = sh_dn;
        for (int c = 0; c < 4; ++c) {
            int vg[4], vd[4], sg = 0, sd = 0;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int e = 4 * l + j;
                const bool in = e < E && cls[e] == c;
                vg[j] = in ? nu_gu[e] : 0;
                vd[j] = in ? nu_dn[e] : 0;
                sg += vg[j];
                sd += vd[j];
            }
            int ig = sg, id = sd;
#pragma unroll
            for (int o = 1; o < 64; o <<= 1) {
                const int tg = __shfl_up(ig, o), td = __shfl_up(id, o);
                if (l >= o) {
                    ig += tg;
                    id += td;
                }
            }
            int rg = bg + ig - sg, rd = bd + id - sd;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int e = 4 * l + j;
                if (e < E && cls[e] == c) {
                    base_gu[e] = rg;
                    base_dn[e] = rd;
                }
                rg += vg[j];
                rd += vd[j];
            }
            bg += __shfl(ig, 63);
            bd += __shfl(id, 63);
        }
        if (l == 0) {
            tot[0] = bg;
            tot[1] = bd;
        }
    }
    __syncthreads();
}

__device__ __forceinline__ int width_class(int bits) { return bits == 8 ? 0 : bits == 4 ? 1 : bits == 3 ? 2 : 3; }

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

// tiled units of expert e (c slots from slot st): chunks of tiled_per(c) slots, each split into `split` ranges
// of row blocks (Item.rb = first | count << 16)
__device__ __forceinline__ int rb_range(int R, int split, int r) { return (r * (R / split)) | ((R / split) << 16); }
__device__ void emit_tiled_units(int e, int c, int st, int bits, int split, int base_gu, int base_dn, Item* tunits_gu,
                                 Item* tunits_dn) {
    const int nch = tiled_chunks(c), per = tiled_per(c);
    const int rg = tiled_row_blocks(false, bits), rd = tiled_row_blocks(true, bits);
    for (int j = 0; j < nch; ++j) {
        const int s0 = st + j * per, n = min(per, c - j * per);
        for (int r = 0; r < split; ++r) {
            tunits_gu[base_gu + j * split + r] = Item{e, s0, n, rb_range(rg, split, r)};
            tunits_dn[base_dn + j * split + r] = Item{e, s0, n, rb_range(rd, split, r)};
        }
    }
}

// the shared expert's tiled units (all T tokens, slots T K + t), the first of both tiled lists
__device__ void emit_shared_tiled_units(int E, int T, int K, int bits, int split, Item* tunits_gu, Item* tunits_dn) {
    const int nch = tiled_chunks(T), per = tiled_per(T);
    const int rg = tiled_row_blocks(false, bits), rd = tiled_row_blocks(true, bits);
    for (int u = threadIdx.x; u < nch * split; u += blockDim.x) {
        const int j = u / split, r = u % split;
        const Item it{E, T * K + j * per, min(per, T - j * per), 0};
        tunits_gu[u] = Item{it.expert, it.slot0, it.ntok, rb_range(rg, split, r)};
        tunits_dn[u] = Item{it.expert, it.slot0, it.ntok, rb_range(rd, split, r)};
    }
}

struct DispatchOut {         // written by the single-block fused route (decode): the plan + place results
    int has_shared, ntok;
    const int8_t* bits;      // code width per expert [E + 1] (orders and splits the work units)
    int* count;
    int* start;
    Item* units_gu;
    Item* units_dn;
    int* n_units;
    int* slot_token;
    float* slot_weight;
    int* tok_slots;
};

constexpr int RT_THREADS = 1024;

// One routing block per workgroup (engine/ops.cu:256-327, quant/s03_teacher_pass.py:132-146):
//   logit = sum of the nchunks partials (c ascending); score = sigmoid(logit); s = score + bias;
//   pool = top-C experts by max over the block's tokens of s, ranked (value desc, index asc) (C >= E: all);
//   per token top-K of s in the pool, (value desc, index asc): 8 lanes per token each keep a sorted top-8 of
//   their 32 experts, then three xor-shuffle merges give every lane the token's top-8;
//   w_k = score_k / (sum_k score_k + 1e-20) * rscale, the sum in rank order.
// Writes topk/topw [T, K] and mask[block, e] = bit t of the block's tokens that picked e. FUSED (T <= block, the
// decode step, engine/ops.cu:333-370): the same workgroup also builds the slots and work items.
// 1024 threads: every partial of the block is loaded in one batch.
template <bool FUSED>
__global__ void __launch_bounds__(RT_THREADS) route_kernel(const float* __restrict__ part, int nchunks,
                                                           const float* __restrict__ bias, int T, int E, int K, int C,
                                                           int block, float rscale, int* __restrict__ topk,
                                                           float* __restrict__ topw, uint32_t* __restrict__ mask,
                                                           DispatchOut dout) {
    __shared__ float sig[MAXB][MAXE + 1];
    __shared__ uint64_t key[MAXE];
    __shared__ float sbias[MAXE];
    __shared__ int inpool[MAXE];
    __shared__ uint32_t tmask[MAXE];
    __shared__ int sstart[MAXE];
    __shared__ int cnt[MAXE];
    __shared__ int nits[MAXE];
    __shared__ int ibase[MAXE];
    __shared__ int tots[2];
    __shared__ int wcls[MAXE];
    __shared__ int nu_gu[MAXE], nu_dn[MAXE], ub_gu[MAXE], ub_dn[MAXE], utot[2];
    const int b = blockIdx.x, t0 = b * block, tb = min(block, T - t0), tid = threadIdx.x;
    if (tid < E) {
        sbias[tid] = bias[tid];
        tmask[tid] = 0u;
    }
    {   // logits: positions (token, 4 experts), <= 2 per thread, all chunks loaded before any is summed
        const int E4 = E / 4, npos = tb * E4;
        float4 p[2][ROUTER_KC];
#pragma unroll
        for (int r = 0; r < 2; ++r) {
            const int pos = tid + r * RT_THREADS, t = pos / E4, e4 = pos % E4;
#pragma unroll
            for (int c = 0; c < ROUTER_KC; ++c)
                if (pos < npos && c < nchunks)
                    p[r][c] = *reinterpret_cast<const float4*>(part + (size_t(c) * T + t0 + t) * E + 4 * e4);
        }
#pragma unroll
        for (int r = 0; r < 2; ++r) {
            const int pos = tid + r * RT_THREADS, t = pos / E4, e4 = pos % E4;
            if (pos < npos) {
                float4 l = p[r][0];
#pragma unroll
                for (int c = 1; c < ROUTER_KC; ++c) {
                    if (c < nchunks) {
                        l.x = l.x + p[r][c].x;
                        l.y = l.y + p[r][c].y;
                        l.z = l.z + p[r][c].z;
                        l.w = l.w + p[r][c].w;
                    }
                }
                sig[t][4 * e4] = sigmoid_f32(l.x);
                sig[t][4 * e4 + 1] = sigmoid_f32(l.y);
                sig[t][4 * e4 + 2] = sigmoid_f32(l.z);
                sig[t][4 * e4 + 3] = sigmoid_f32(l.w);
            }
        }
    }
    __syncthreads();
    if (C < E) {
        if (tid < E) {
            float km = -__builtin_inff();
            for (int t = 0; t < tb; ++t) km = fmaxf(km, sig[t][tid] + sbias[tid]);
            key[tid] = sel_key(km, tid);
        }
        __syncthreads();
    }
    if (tid < E) {   // pool = the C largest keys: rank = number of larger keys
        int rank = 0;
        if (C < E) {
            const uint64_t ke = key[tid];
#pragma unroll 8
            for (int j = 0; j < E; ++j) rank += key[j] > ke;
        }
        inpool[tid] = rank < C;
    }
    __syncthreads();
    // selection: 32 lanes per token (all 1024 threads), 8 candidates per lane read before use and sorted, then
    // five xor-shuffle merges (1 .. 16) give every lane of the token its best 8
    const int tl = tid >> 5, sub = tid & 31;
    uint64_t best[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        const int ex = sub * 8 + j;
        const bool ok = tl < tb && ex < E && inpool[ex];
        best[j] = ok ? sel_key(sig[tl][ex] + sbias[ex], ex) : 0ull;
    }
    sort8(best);
#pragma unroll 1
    for (int o = 1; o < 32; o <<= 1) {
        uint64_t other[8];
#pragma unroll
        for (int k = 0; k < 8; ++k) other[k] = shfl_xor64(best[k], o);
        merge8(best, other);
    }
    int bi[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) bi[k] = key_index(best[k]);
    float mine = 0.0f, wsum = 0.0f;
    int mysel = 0;
    const bool owner = tl < tb && sub < K;
    if (tl < tb) {
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            if (k < K) {
                const float sk = sig[tl][bi[k]];
                wsum = wsum + sk;
                if (k == sub) {
                    mine = sk;
                    mysel = bi[k];
                }
            }
        }
        if (owner) {
            topk[size_t(t0 + tl) * K + sub] = mysel;
            topw[size_t(t0 + tl) * K + sub] = mine / (wsum + 1e-20f) * rscale;
            atomicOr(&tmask[mysel], 1u << tl);
        }
    }
    __syncthreads();
    if (tid < E) mask[size_t(b) * E + tid] = tmask[tid];
    if constexpr (FUSED) {
        // one block: slot ranges = exclusive scan of the per-expert token counts; work units (items of <= ntok
        // slots, split into row blocks by code width) ordered heaviest first
        const int ns = dout.has_shared ? (T + dout.ntok - 1) / dout.ntok : 0;
        const int sbits = dout.has_shared ? dout.bits[E] : 8;
        if (tid < E) {
            const int c = __popc(tmask[tid]);
            const int b = dout.bits[tid];
            const int nit = (c + dout.ntok - 1) / dout.ntok;
            cnt[tid] = c;
            nits[tid] = nit;
            nu_gu[tid] = nit * gemm_row_blocks(false, b);
            nu_dn[tid] = nit * gemm_row_blocks(true, b);
            wcls[tid] = width_class(b);
        }
        __syncthreads();
        expert_scan2(cnt, nits, E, sstart, ibase, tots);
        unit_offsets(nu_gu, nu_dn, wcls, E, ns * gemm_row_blocks(false, sbits), ns * gemm_row_blocks(true, sbits),
                     ub_gu, ub_dn, utot);
        if (tid < E) {
            dout.count[tid] = cnt[tid];
            dout.start[tid] = sstart[tid];
            emit_units(tid, cnt[tid], sstart[tid], dout.ntok, dout.bits[tid], ub_gu[tid], ub_dn[tid], dout.units_gu,
                       dout.units_dn);
        }
        if (ns) emit_shared_units(E, T, K, dout.ntok, sbits, dout.units_gu, dout.units_dn);
        if (tid == 0) {
            dout.n_units[0] = utot[0];
            dout.n_units[1] = utot[1];
        }
        __syncthreads();
        if (owner) {
            const int t = t0 + tl;
            const int sl = sstart[mysel] + __popc(tmask[mysel] & ((1u << tl) - 1u));
            dout.slot_token[sl] = t;
            dout.slot_weight[sl] = mine / (wsum + 1e-20f) * rscale;
            dout.tok_slots[size_t(t) * (K + 1) + sub] = sl;
        }
        if (tid < tb) {
            const int t = t0 + tid;
            if (dout.has_shared) {
                dout.slot_token[T * K + t] = t;
                dout.slot_weight[T * K + t] = 1.0f;
            }
            dout.tok_slots[size_t(t) * (K + 1) + K] = dout.has_shared ? T * K + t : -1;
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
// One workgroup, thread = expert.
__global__ void __launch_bounds__(256) plan_kernel(const uint32_t* __restrict__ mask, int T, int E, int K, int block,
                                                   int has_shared, int ntok, int tiled,
                                                   const int8_t* __restrict__ bits, int* __restrict__ count,
                                                   int* __restrict__ start, int* __restrict__ bpre,
                                                   Item* __restrict__ units_gu, Item* __restrict__ units_dn,
                                                   Item* __restrict__ tunits_gu, Item* __restrict__ tunits_dn,
                                                   int* __restrict__ n_units) {
    __shared__ int buf[256];
    __shared__ int nu_gu[MAXE], nu_dn[MAXE], ub_gu[MAXE], ub_dn[MAXE], wcls[MAXE], utot[2];
    __shared__ int tu_gu[MAXE], tu_dn[MAXE], tb_gu[MAXE], tb_dn[MAXE], ttot[2];
    const int e = threadIdx.x, nb = (T + block - 1) / block;
    int c = 0;
    if (e < E)
        for (int b = 0; b < nb; ++b) c += __popc(mask[size_t(b) * E + e]);
    int tot_slots;
    const int st = block_excl_scan<256>(c, buf, &tot_slots);
    const bool big = tiled && c > TILED_MIN;
    const bool sbig = has_shared && tiled && T > TILED_MIN;
    const int nsch = sbig ? tiled_chunks(T) : 0;
    // row-block ranges per chunk: enough tiled units to fill the GPU (split a chunk's rows when chunks are few)
    int all_chunks;
    block_excl_scan<256>(e < E && big ? tiled_chunks(c) : 0, buf, &all_chunks);
    all_chunks += nsch;
    const int split = all_chunks >= 384 ? 1 : all_chunks >= 192 ? 2 : 4;
    if (e < E) {
        const int bw = bits[e];
        const int nit = big ? 0 : (c + ntok - 1) / ntok, nch = big ? tiled_chunks(c) : 0;
        nu_gu[e] = nit * gemm_row_blocks(false, bw);
        nu_dn[e] = nit * gemm_row_blocks(true, bw);
        tu_gu[e] = nch * split;
        tu_dn[e] = nch * split;
        wcls[e] = width_class(bw);
    }
    __syncthreads();
    const int sbits = has_shared ? bits[E] : 8;
    const int ns = has_shared && !sbig ? (T + ntok - 1) / ntok : 0;
    unit_offsets(nu_gu, nu_dn, wcls, E, ns * gemm_row_blocks(false, sbits), ns * gemm_row_blocks(true, sbits), ub_gu,
                 ub_dn, utot);
    unit_offsets(tu_gu, tu_dn, wcls, E, nsch * split, nsch * split, tb_gu, tb_dn, ttot);
    if (e < E) {
        count[e] = c;
        start[e] = st;
        int run = st;
        for (int b = 0; b < nb; ++b) {
            bpre[size_t(b) * E + e] = run;
            run += __popc(mask[size_t(b) * E + e]);
        }
        if (big) emit_tiled_units(e, c, st, bits[e], split, tb_gu[e], tb_dn[e], tunits_gu, tunits_dn);
        else emit_units(e, c, st, ntok, bits[e], ub_gu[e], ub_dn[e], units_gu, units_dn);
    }
    if (ns) emit_shared_units(E, T, K, ntok, sbits, units_gu, units_dn);
    if (sbig) emit_shared_tiled_units(E, T, K, sbits, split, tunits_gu, tunits_dn);
    if (threadIdx.x == 0) {
        n_units[0] = utot[0];
        n_units[1] = utot[1];
        n_units[2] = ttot[0];
        n_units[3] = ttot[1];
    }
}

// Place every (token, k) pair in its slot; tok_slots[t, K] = the shared slot (or -1). grid nb, 256 threads.
__global__ void __launch_bounds__(256) place_kernel(const int* __restrict__ topk, const float* __restrict__ topw,
                                                    const uint32_t* __restrict__ mask, const int* __restrict__ bpre,
                                                    int T, int E, int K, int block, int has_shared,
                                                    int* __restrict__ slot_token, float* __restrict__ slot_weight,
                                                    int* __restrict__ tok_slots) {
    const int b = blockIdx.x, t0 = b * block, tb = min(block, T - t0);
    for (int p = threadIdx.x; p < tb * K; p += blockDim.x) {
        const int tl = p / K, k = p % K, t = t0 + tl;
        const int ex = topk[size_t(t) * K + k];
        const uint32_t m = mask[size_t(b) * E + ex];
        const int sl = bpre[size_t(b) * E + ex] + __popc(m & ((1u << tl) - 1u));
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
}

}  // namespace

hipError_t launch_router_logits(const float* x, const float* Wr, int T, int H, int E, float* part, hipStream_t st) {
    static bool attr = false;
    if (!attr) {
        const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(router_logits_kernel),
                                                 hipFuncAttributeMaxDynamicSharedMemorySize, ROUTER_LDS);
        if (e != hipSuccess) return e;
        attr = true;
    }
    const dim3 grid(E / 64, (T + 31) / 32, ROUTER_KC);
    router_logits_kernel<<<grid, 256, ROUTER_LDS, st>>>(x, Wr, T, H, E, part);
    return hipGetLastError();
}

hipError_t launch_route(const float* part, int nchunks, const float* bias, int T, int E, int K, int C, int block,
                        float rscale, int32_t* topk, float* topw, uint32_t* mask, hipStream_t st) {
    const int nb = (T + block - 1) / block;
    route_kernel<false><<<nb, RT_THREADS, 0, st>>>(part, nchunks, bias, T, E, K, C, block, rscale, topk, topw, mask,
                                                   DispatchOut{});
    return hipGetLastError();
}

hipError_t launch_route_dispatch(const float* part, int nchunks, const float* bias, int T, int E, int K, int C,
                                 int block, float rscale, int32_t* topk, float* topw, uint32_t* mask, int has_shared,
                                 int ntok, const int8_t* bits, int32_t* count, int32_t* start, Item* units_gu,
                                 Item* units_dn, int* n_units, int32_t* slot_token, float* slot_weight,
                                 int32_t* tok_slots, hipStream_t st) {
    if (T > block) return hipErrorInvalidValue;
    const DispatchOut d{has_shared, ntok, bits, count, start, units_gu, units_dn, n_units, slot_token, slot_weight,
                        tok_slots};
    route_kernel<true><<<1, RT_THREADS, 0, st>>>(part, nchunks, bias, T, E, K, C, block, rscale, topk, topw, mask, d);
    return hipGetLastError();
}

hipError_t launch_masks(const int32_t* topk, int T, int E, int K, int block, uint32_t* mask, hipStream_t st) {
    const int nb = (T + block - 1) / block;
    masks_kernel<<<nb, 256, 0, st>>>(topk, T, E, K, block, mask);
    return hipGetLastError();
}

hipError_t launch_plan(const uint32_t* mask, int T, int E, int K, int block, int has_shared, int ntok, int tiled,
                       const int8_t* bits, int32_t* count, int32_t* start, int32_t* bpre, Item* units_gu,
                       Item* units_dn, Item* tunits_gu, Item* tunits_dn, int* n_units, hipStream_t st) {
    plan_kernel<<<1, 256, 0, st>>>(mask, T, E, K, block, has_shared, ntok, tiled, bits, count, start, bpre, units_gu,
                                   units_dn, tunits_gu, tunits_dn, n_units);
    return hipGetLastError();
}

hipError_t launch_place(const int32_t* topk, const float* topw, const uint32_t* mask, const int32_t* bpre, int T,
                        int E, int K, int block, int has_shared, int32_t* slot_token, float* slot_weight,
                        int32_t* tok_slots, hipStream_t st) {
    const int nb = (T + block - 1) / block;
    place_kernel<<<nb, 256, 0, st>>>(topk, topw, mask, bpre, T, E, K, block, has_shared, slot_token, slot_weight,
                                     tok_slots);
    return hipGetLastError();
}

}  // namespace llmoe
