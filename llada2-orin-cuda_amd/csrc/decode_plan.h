// The decode step's slot plan (one routing block, T <= 32, engine/ops.cu:333-370), as device functions shared by
// the dispatch kernel (route.hip) and the gate_up GEMM that plans for itself (expert_gemm.hip).
//
// Input: tmask[e], bit t set when token t picked expert e (written by the selection kernel), and the code width of
// each expert. Slots are expert-major and token-ascending (expert e's slots start at the count prefix of the
// experts before it); the shared expert's slots are T K + t. Work units are items of <= 16 slots split into row
// blocks by code width, ordered by class -- 2, 3, 4, 8-bit experts (expert order within a class), then the shared
// expert's -- so the longest units start first.
//
// Every workgroup of 256 threads can build the plan in LDS (one thread per expert: three scans), and any of them
// can then name unit u of the gate_up list without the list in memory: the class from the class totals, the
// expert by binary search on the class's inclusive scan, then the item and row block.
#pragma once
#include "llmoe_internal.h"

namespace llmoe {

constexpr int PLAN_MAXE = 256;   // experts: one thread each

struct DispatchOut {         // the plan and placement written for the down GEMM, the combine and the buffers' readers
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

struct DecodeState {
    uint32_t* blockmax;   // [E] ordered keys of max_t (sigmoid + bias)
    uint32_t* tmask;      // [E] bit t: token t picked the expert
};

__device__ __forceinline__ int decode_class(int bits) { return bits == 2 ? 0 : bits == 3 ? 1 : bits == 4 ? 2 : 3; }

// shared-expert unit u of a list with r row blocks per item (items of 16 slots at T K + 16 j)
__device__ __forceinline__ Item unit_shared(int u, int r, int E, int T, int K) {
    const int j = u / r;
    return Item{E, T * K + 16 * j, min(16, T - 16 * j), u % r};
}

__device__ __forceinline__ int class_field(uint64_t v, int k) { return int((v >> (16 * k)) & 0xFFFFu); }

struct DecodePlan {            // LDS
    uint32_t m[PLAN_MAXE];     // token masks
    int start[PLAN_MAXE];      // first slot of each expert
    uint64_t ig[PLAN_MAXE];    // inclusive scans of the gate_up / down unit counts: 4 classes x 16 bits
    uint64_t id[PLAN_MAXE];
    int8_t bits[PLAN_MAXE];
    uint64_t totg, totd;       // class totals
    int wt_i[4];
    uint64_t wt_g[4], wt_d[4];
};

// One thread per expert (blockDim 256, E <= 256): P filled, then a barrier. Returns this thread's token mask.
__device__ __forceinline__ uint32_t decode_plan_scan(int E, const uint32_t* __restrict__ tmask,
                                                     const int8_t* __restrict__ bits, DecodePlan& P) {
    const int e = threadIdx.x, lane = e & 63, w = e >> 6;
    const uint32_t m = e < E ? tmask[e] : 0u;
    const int bw = e < E ? bits[e] : 2;
    const int c = __popc(m), nit = (c + 15) >> 4, cls = decode_class(bw);
    const uint64_t vg = uint64_t(nit * gemm_row_blocks(false, bw)) << (16 * cls);
    const uint64_t vd = uint64_t(nit * gemm_row_blocks(true, bw)) << (16 * cls);
    // three inclusive scans over the 256 threads in one pass: wave shuffles, then the wave totals
    int incl = wave_incl_scan(c);
    uint64_t ig = wave_incl_scan(vg), id = wave_incl_scan(vd);
    if (lane == 63) {
        P.wt_i[w] = incl;
        P.wt_g[w] = ig;
        P.wt_d[w] = id;
    }
    __syncthreads();
    for (int i = 0; i < w; ++i) {
        incl += P.wt_i[i];
        ig += P.wt_g[i];
        id += P.wt_d[i];
    }
    P.m[e] = m;
    P.start[e] = incl - c;
    P.ig[e] = ig;
    P.id[e] = id;
    P.bits[e] = int8_t(bw);
    if (e == 255) {
        P.totg = ig;
        P.totd = id;
    }
    __syncthreads();
    return m;
}

// total units of the gate_up (down) list
__device__ __forceinline__ int decode_plan_units(const DecodePlan& P, bool down, int T, int has_shared, int sbits) {
    const uint64_t tot = down ? P.totd : P.totg;
    const int ns = has_shared ? (T + 15) >> 4 : 0;
    return class_field(tot, 0) + class_field(tot, 1) + class_field(tot, 2) + class_field(tot, 3) +
           ns * gemm_row_blocks(down, sbits);
}

// Unit u of the gate_up (down) list, from the plan alone (the same unit the dispatch writes at position u).
__device__ __forceinline__ Item decode_plan_unit(const DecodePlan& P, bool down, int u, int T, int E, int K,
                                                 int sbits) {
    const uint64_t tot = down ? P.totd : P.totg;
    const uint64_t* scan = down ? P.id : P.ig;
    int base = 0;
    for (int k = 0; k < 4; ++k) {
        const int cnt = class_field(tot, k);
        if (u < base + cnt) {
            const int v = u - base;
            int lo = 0, hi = E - 1;   // the first expert whose inclusive class-k count exceeds v
            while (lo < hi) {
                const int mid = (lo + hi) >> 1;
                if (class_field(scan[mid], k) > v) hi = mid;
                else lo = mid + 1;
            }
            const int e = lo, bw = P.bits[e], c = __popc(P.m[e]);
            const int rb = gemm_row_blocks(down, bw), nit = (c + 15) >> 4;
            const int off = v - (class_field(scan[e], k) - nit * rb), j = off / rb;
            return Item{e, P.start[e] + 16 * j, min(16, c - 16 * j), off % rb};
        }
        base += cnt;
    }
    return unit_shared(u - base, gemm_row_blocks(down, sbits), E, T, K);
}

// The written part of the plan. decode_plan_write_expert: expert e's count, start and units of both lists, by the
// threads i0, i0 + stride, ... decode_plan_write_rest: the shared expert's units and slots, the unit counts, and the
// placement of every (token, k) pair, by the threads tid, tid + stride, ... P from decode_plan_scan.
__device__ __forceinline__ void decode_plan_write_expert(const DecodePlan& P, int e, int i0, int stride,
                                                         const DispatchOut& d) {
    const int bw = P.bits[e], c = __popc(P.m[e]), cls = decode_class(bw), nit = (c + 15) >> 4;
    const int rg = gemm_row_blocks(false, bw), rd = gemm_row_blocks(true, bw);
    // list positions: the totals of the classes before this one, plus the expert's exclusive count in its class
    int bg = 0, bd = 0;
    for (int k = 0; k < cls; ++k) {
        bg += class_field(P.totg, k);
        bd += class_field(P.totd, k);
    }
    const int og = bg + class_field(P.ig[e], cls) - nit * rg, od = bd + class_field(P.id[e], cls) - nit * rd;
    if (i0 == 0) {
        d.count[e] = c;
        d.start[e] = P.start[e];
    }
    for (int i = i0; i < nit * rg; i += stride) {
        const int j = i / rg;
        d.units_gu[og + i] = Item{e, P.start[e] + 16 * j, min(16, c - 16 * j), i % rg};
    }
    for (int i = i0; i < nit * rd; i += stride) {
        const int j = i / rd;
        d.units_dn[od + i] = Item{e, P.start[e] + 16 * j, min(16, c - 16 * j), i % rd};
    }
}

__device__ __forceinline__ void decode_plan_write_rest(const DecodePlan& P, int tid, int stride, int T, int E, int K,
                                                       const int* __restrict__ topk, const float* __restrict__ topw,
                                                       const DispatchOut& d) {
    const int sbits = d.has_shared ? d.bits[E] : 8;
    const int ns = d.has_shared ? (T + 15) >> 4 : 0;
    int bg = 0, bd = 0;
    for (int k = 0; k < 4; ++k) {
        bg += class_field(P.totg, k);
        bd += class_field(P.totd, k);
    }
    const int srg = gemm_row_blocks(false, sbits), srd = gemm_row_blocks(true, sbits);
    for (int u = tid; u < ns * srg; u += stride) d.units_gu[bg + u] = unit_shared(u, srg, E, T, K);
    for (int u = tid; u < ns * srd; u += stride) d.units_dn[bd + u] = unit_shared(u, srd, E, T, K);
    if (tid == 0) {
        d.n_units[0] = bg + ns * srg;
        d.n_units[1] = bd + ns * srd;
        d.n_units[2] = 0;
        d.n_units[3] = 0;
    }
    // place every (token, k) pair: slot = the expert's start + the tokens before t that picked it
    for (int p = tid; p < T * K; p += stride) {
        const int t = p / K, ex = topk[p];
        const int sl = P.start[ex] + __popc(P.m[ex] & ((1u << t) - 1u));
        d.slot_token[sl] = t;
        d.slot_weight[sl] = topw[p];
        d.tok_slots[p + t] = sl;                      // [t][k] of the [T][K + 1] table
    }
    for (int t = tid; t < T; t += stride) {
        if (d.has_shared) {
            d.slot_token[T * K + t] = t;
            d.slot_weight[T * K + t] = 1.0f;
        }
        d.tok_slots[size_t(t) * (K + 1) + K] = d.has_shared ? T * K + t : -1;
    }
}

struct DecodePlanArgs {   // the self-planning gate_up GEMM's routing inputs and plan outputs
    int T, E, K;
    const uint32_t* tmask;
    uint32_t* tcopy;     // [E] the masks planned from, kept for a re-launch (the down GEMM zeroes tmask)
    const int32_t* topk;
    const float* topw;
    DispatchOut d;
    const uint64_t* d_off;   // [E + 1] down matrix offsets (the down units' weights requested ahead)
    int pf_bytes;            // bytes of each down unit requested by the workgroups with no second gate_up unit
};

// the token of slot (it.slot0 + n) of a decode unit, from the plan: the (16 j + n)-th token of the expert's mask for
// a routed expert, t = slot - T K for the shared expert
__device__ __forceinline__ int decode_slot_token(const DecodePlan& P, const Item& it, int n, int T, int K, int E) {
    if (it.expert >= E) return it.slot0 + n - T * K;
    uint32_t m = P.m[it.expert];
    for (int i = it.slot0 + n - P.start[it.expert]; i > 0; --i) m &= m - 1u;
    return __builtin_ctz(m);
}

}  // namespace llmoe
