// Router and dispatch kernels (engine/ops.cu:137-423): router logits, per-block sigmoid+bias scoring with the
// block expert pool and per-token top-K, routing weights, and the deterministic counting sort of (token, k)
// pairs into expert-major slots with the GEMM work items. All counts stay on the device.
#include "llmoe_internal.h"

namespace llmoe {

namespace {

constexpr int MAXB = 32;    // tokens per routing block (one 32-bit token mask per expert)
constexpr int MAXE = 256;   // experts (one thread each)

// logits partial c: fma chain over k = c H/8 .. (c+1) H/8 - 1 ascending from 0 (the summation order is fixed so
// the CPU checker reproduces it). Tile 32 tokens x 64 experts per workgroup, 2 x 4 outputs per thread.
// grid (E/64, ceil(T/32), 8), 256 threads.
__global__ void __launch_bounds__(256) router_logits_kernel(const float* __restrict__ x, const float* __restrict__ Wr,
                                                            int T, int H, int E, float* __restrict__ part) {
    __shared__ float xs[32][33];
    __shared__ float ws[32][64];
    const int e0 = blockIdx.x * 64, t0 = blockIdx.y * 32, c = blockIdx.z, KW = H / ROUTER_KC, kb = c * KW;
    const int tid = threadIdx.x, ty = tid >> 4, tx = tid & 15;
    float acc[2][4] = {{0.0f, 0.0f, 0.0f, 0.0f}, {0.0f, 0.0f, 0.0f, 0.0f}};
    for (int k0 = kb; k0 < kb + KW; k0 += 32) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int idx = tid + 256 * i, t = idx >> 5, k = idx & 31;
            xs[k][t] = t0 + t < T ? x[size_t(t0 + t) * H + k0 + k] : 0.0f;
        }
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const int idx = tid + 256 * i, k = idx >> 6, e = idx & 63;
            ws[k][e] = Wr[size_t(k0 + k) * E + e0 + e];
        }
        __syncthreads();
#pragma unroll 8
        for (int kk = 0; kk < 32; ++kk) {
            const float xa = xs[kk][2 * ty], xb = xs[kk][2 * ty + 1];
            const float4 w = *reinterpret_cast<const float4*>(&ws[kk][4 * tx]);
            const float wv[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                acc[0][j] = __builtin_fmaf(xa, wv[j], acc[0][j]);
                acc[1][j] = __builtin_fmaf(xb, wv[j], acc[1][j]);
            }
        }
        __syncthreads();
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

// One routing block per workgroup, thread = expert (engine/ops.cu:256-327, quant/s03_teacher_pass.py:132-146):
//   logit = sum of the nchunks partials (c ascending); score = sigmoid(logit); s = score + bias;
//   pool = top-C experts by max over the block's tokens of s, ranked (value desc, index asc) (C >= E: all);
//   per token top-K of s in the pool, (value desc, index asc), by K rounds of a wavefront arg-max;
//   w_k = score_k / (sum_k score_k + 1e-20) * rscale.
// Writes topk/topw [T, K] and mask[block, e] = bit t of the block's tokens that picked e.
__global__ void __launch_bounds__(256) route_kernel(const float* __restrict__ part, int nchunks,
                                                    const float* __restrict__ bias, int T, int E, int K, int C,
                                                    int block, float rscale, int* __restrict__ topk,
                                                    float* __restrict__ topw, uint32_t* __restrict__ mask) {
    __shared__ float sig[MAXB][MAXE];
    __shared__ float key[MAXE];
    __shared__ float sbias[MAXE];
    __shared__ int inpool[MAXE];
    __shared__ uint32_t tmask[MAXE];
    const int b = blockIdx.x, t0 = b * block, tb = min(block, T - t0), e = threadIdx.x;
    if (e < E) {
        const float be = bias[e];
        float km = -__builtin_inff();
        for (int t = 0; t < tb; ++t) {
            float l = part[size_t(t0 + t) * E + e];
            for (int c = 1; c < nchunks; ++c) l = l + part[(size_t(c) * T + t0 + t) * E + e];
            const float sg = sigmoid_f32(l);
            sig[t][e] = sg;
            km = fmaxf(km, sg + be);
        }
        key[e] = km;
        sbias[e] = be;
        tmask[e] = 0u;
    }
    __syncthreads();
    if (e < E) {
        int rank = 0;
        if (C < E) {
            const float ke = key[e];
            for (int j = 0; j < E; ++j) rank += beats(key[j], j, ke, e);
        }
        inpool[e] = rank < C;
    }
    __syncthreads();
    const int lane = e & 63, wave = e >> 6;
    for (int t = wave; t < tb; t += 4) {
        float v[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int ex = lane + 64 * j;
            v[j] = (ex < E && inpool[ex]) ? sig[t][ex] + sbias[ex] : -__builtin_inff();
        }
        int taken = 0, mysel = -1;
        float mysig = 0.0f, wsum = 0.0f;
        for (int k = 0; k < K; ++k) {
            float bv = -__builtin_inff();
            int bi = 0x7fffffff;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int ex = lane + 64 * j;
                if (!((taken >> j) & 1) && ex < E && beats(v[j], ex, bv, bi)) {
                    bv = v[j];
                    bi = ex;
                }
            }
#pragma unroll
            for (int o = 32; o > 0; o >>= 1) {
                const float ov = __shfl_xor(bv, o);
                const int oi = __shfl_xor(bi, o);
                if (beats(ov, oi, bv, bi)) {
                    bv = ov;
                    bi = oi;
                }
            }
            if ((bi & 63) == lane) taken |= 1 << (bi >> 6);
            const float sk = sig[t][bi];
            wsum = wsum + sk;
            if (lane == k) {
                mysel = bi;
                mysig = sk;
            }
        }
        if (lane < K) {
            topk[size_t(t0 + t) * K + lane] = mysel;
            topw[size_t(t0 + t) * K + lane] = mysig / (wsum + 1e-20f) * rscale;
            atomicOr(&tmask[mysel], 1u << t);
        }
    }
    __syncthreads();
    if (e < E) mask[size_t(b) * E + e] = tmask[e];
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

// exclusive prefix sum over the 256 threads of a block (Hillis-Steele in LDS); *total = the full sum
__device__ int block_excl_scan(int v, int* buf, int* total) {
    const int i = threadIdx.x;
    buf[i] = v;
    __syncthreads();
    for (int o = 1; o < 256; o <<= 1) {
        const int add = i >= o ? buf[i - o] : 0;
        __syncthreads();
        buf[i] += add;
        __syncthreads();
    }
    const int incl = buf[i];
    *total = buf[255];
    __syncthreads();
    return incl - v;
}

// Slot ranges and work items (engine/ops.cu:333-370, :384-410): slots expert-major (expert ascending), inside
// an expert block-major then token-ascending; items of <= ntok slots per expert; shared-expert items last.
// One workgroup, thread = expert.
__global__ void __launch_bounds__(256) plan_kernel(const uint32_t* __restrict__ mask, int T, int E, int K, int block,
                                                   int has_shared, int ntok, int* __restrict__ count,
                                                   int* __restrict__ start, int* __restrict__ bpre,
                                                   Item* __restrict__ items, int* __restrict__ n_items) {
    __shared__ int buf[256];
    const int e = threadIdx.x, nb = (T + block - 1) / block;
    int c = 0;
    if (e < E)
        for (int b = 0; b < nb; ++b) c += __popc(mask[size_t(b) * E + e]);
    int tot_slots, tot_items;
    const int st = block_excl_scan(c, buf, &tot_slots);
    const int nit = e < E ? (c + ntok - 1) / ntok : 0;
    const int ib = block_excl_scan(nit, buf, &tot_items);
    if (e < E) {
        count[e] = c;
        start[e] = st;
        int run = st;
        for (int b = 0; b < nb; ++b) {
            bpre[size_t(b) * E + e] = run;
            run += __popc(mask[size_t(b) * E + e]);
        }
        for (int j = 0; j < nit; ++j) {
            const int n = min(ntok, c - j * ntok);
            items[ib + j] = Item{e, st + j * ntok, n, 0};
        }
    }
    const int ns = has_shared ? (T + ntok - 1) / ntok : 0;
    for (int j = threadIdx.x; j < ns; j += blockDim.x)
        items[tot_items + j] = Item{E, T * K + j * ntok, min(ntok, T - j * ntok), 0};
    if (threadIdx.x == 0) *n_items = tot_items + ns;
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
    const dim3 grid(E / 64, (T + 31) / 32, ROUTER_KC);
    router_logits_kernel<<<grid, 256, 0, st>>>(x, Wr, T, H, E, part);
    return hipGetLastError();
}

hipError_t launch_route(const float* part, int nchunks, const float* bias, int T, int E, int K, int C, int block,
                        float rscale, int32_t* topk, float* topw, uint32_t* mask, hipStream_t st) {
    const int nb = (T + block - 1) / block;
    route_kernel<<<nb, 256, 0, st>>>(part, nchunks, bias, T, E, K, C, block, rscale, topk, topw, mask);
    return hipGetLastError();
}

hipError_t launch_masks(const int32_t* topk, int T, int E, int K, int block, uint32_t* mask, hipStream_t st) {
    const int nb = (T + block - 1) / block;
    masks_kernel<<<nb, 256, 0, st>>>(topk, T, E, K, block, mask);
    return hipGetLastError();
}

hipError_t launch_plan(const uint32_t* mask, int T, int E, int K, int block, int has_shared, int ntok,
                       int32_t* count, int32_t* start, int32_t* bpre, Item* items, int* n_items, hipStream_t st) {
    plan_kernel<<<1, 256, 0, st>>>(mask, T, E, K, block, has_shared, ntok, count, start, bpre, items, n_items);
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
