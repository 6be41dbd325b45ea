// libllmoe C ABI (include/llmoe.h): layer construction, workspace, and the launch sequence of the MoE layer
//   A8(x) -> router logits -> route (pool, top-K, weights) -> plan + place (slots, work items)
//   -> gate_up GEMM -> FWHT-512 + A8 -> down GEMM -> combine
// everything asynchronous on the caller's stream (engine/engine.cu:445-479 is the reference sequence).
#include <algorithm>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <new>
#include <set>
#include <string>
#include <vector>

#include "llmoe.h"
#include "decode_plan.h"

using namespace llmoe;

namespace {

// bytes of each down unit the decode gate_up GEMM requests ahead when its units fit one round
constexpr int DOWN_PF_BYTES = 48 * 1024;

thread_local std::string g_err;

int fail(int code, const char* fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof(buf), fmt, ap);
    va_end(ap);
    g_err = buf;
    return code;
}

#define HIPCHECK(expr)                                                                                     \
    do {                                                                                                   \
        const hipError_t e_ = (expr);                                                                      \
        if (e_ != hipSuccess) return fail(LLMOE_EHIP, "%s: %s (%s:%d)", #expr, hipGetErrorString(e_),      \
                                          __FILE__, __LINE__);                                             \
    } while (0)

hipError_t g_setup = hipErrorNotInitialized;
bool g_setup_done = false;

}  // namespace

namespace llmoe {
int tile_wbytes(int bits) { return bits == 8 ? 2048 : bits == 4 ? 1024 : bits == 3 ? 768 : bits == 2 ? 512 : -1; }
size_t packlib_matrix_bytes(int R, int K, int bits) {
    return size_t(R / 16) * size_t(K / GROUP) * size_t(tile_wbytes(bits) + 48);
}
int set_error(int code, const char* msg) {
    g_err = msg;
    return code;
}
int ensure_gemm_setup() {
    if (!g_setup_done) {
        g_setup = gemm_setup();
        if (g_setup == hipSuccess) g_setup = tiled_setup();
        g_setup_done = true;
    }
    return g_setup == hipSuccess ? LLMOE_OK : fail(LLMOE_EHIP, "gemm_setup: %s", hipGetErrorString(g_setup));
}
}  // namespace llmoe

struct NormOut {            // the combine's fused epilogue (llmoe_experts_norm); h == nullptr: plain combine
    const float* signs;
    float eps;
    float* h;
    int8_t* q;
    float* s;
    int32_t* sum;
};

struct Inter {              // the expert stage's intermediates between the kernels
    uint16_t* Z;            // fp16 SiLU(g) u                 [S, I]
    int8_t* zq;             // A8(Z H512)                     [S, I]
    float* zs;              //                                [S, I / 128]
    int32_t* zsum;          //                                [S, I / 128]
    float* Y;               // weighted expert outputs        [S, H]
};

struct llmoe_layer {
    llmoe_layer_desc d{};
    int nexp = 0;                                   // E + has_shared
    uint8_t* arena = nullptr;
    size_t arena_bytes = 0;
    size_t weight_bytes = 0;                        // distinct matrices
    uint64_t* gu_off_d = nullptr;
    uint64_t* d_off_d = nullptr;
    int8_t* bits_d = nullptr;
    float* router_w = nullptr;
    float* bias = nullptr;
    // workspace
    int8_t* xq = nullptr; float* xs = nullptr; int32_t* xsum = nullptr;
    float* part = nullptr;
    int32_t* topk = nullptr; float* topw = nullptr;
    uint32_t* mask = nullptr; int32_t* bpre = nullptr;
    float* sig = nullptr;                                                          // decode routing scratch
    uint32_t* blockmax = nullptr; uint32_t* tmask = nullptr;                      // zero between calls
    int32_t* count = nullptr; int32_t* start = nullptr;
    Item* units_gu = nullptr; Item* units_dn = nullptr; int* n_units = nullptr;   // streamed GEMM work units
    Item* tunits_gu = nullptr; Item* tunits_dn = nullptr;                          // tiled GEMM work units
    int32_t* slot_token = nullptr; float* slot_weight = nullptr; int32_t* tok_slots = nullptr;
    uint16_t* Z = nullptr; int8_t* zq = nullptr; float* zs = nullptr; int32_t* zsum = nullptr;
    float* Y = nullptr;
    Item* p_item = nullptr; int* p_count = nullptr;  // unit list of llmoe_group_products
    Item p_item_host[MAX_UNITS_PER_ITEM] = {}; int p_count_host = 1;
    size_t items_cap = 0;                           // work items (before the split into row blocks)
    size_t chunks_cap = 0;                          // tiled chunks
    int g_gu = 0, g_dn = 0;                         // tiled GEMM grids (workgroups of the work partition)
    int* tstart = nullptr;                          // [g_gu + 1 + g_dn + 1] tiled work partition
    bool fast = false;                              // numerics: the gate_up SiLU by the hardware transcendentals
    // routing state
    int routed_T = -1, ntok = 16, max_items = 0;
    bool tiled = false;                             // the routing of routed_T may have tiled units
    // a layer forward's decode routing left its masks for the gate_up GEMM to plan from (no dispatch kernel ran):
    // the next expert call plans in its gate_up GEMM and its down GEMM zeroes the masks
    bool plan_pending = false;
    // stage timing
    bool profiling = false;
    hipEvent_t ev[2 * LLMOE_N_STAGES] = {};
    bool ran[LLMOE_N_STAGES] = {};
    // the latest llmoe_experts launch (for llmoe_layer_time_stage)
    GemmArgs last_gu{}, last_dn{}, last_tgu{}, last_tdn{};
    bool last_plan = false;                         // the latest gate_up planned for itself (launch_expert_gemm_plan)
    DecodePlanArgs last_pa{};                       // its arguments, planning from the copy of the masks
    uint32_t* tcopy = nullptr;                      // [E] the masks of the latest self-planned gate_up
    float* last_out = nullptr;
    NormOut last_norm{};
    Inter last_w{};
    int last_S = 0, last_T = 0, last_nt = 1;
    bool last_tiled = false;
    bool last_yhalf = false;                        // the latest call's Y holds fp16 (fast numerics)
    bool have_last = false;
    std::vector<void*> allocs;

    template <class T>
    hipError_t alloc(T** p, size_t count_) {
        void* v = nullptr;
        const hipError_t e = hipMalloc(&v, std::max<size_t>(count_ * sizeof(T), 16));
        if (e == hipSuccess) {
            allocs.push_back(v);
            *p = static_cast<T*>(v);
        }
        return e;
    }
    ~llmoe_layer() {
        for (hipEvent_t e : ev)
            if (e) (void)hipEventDestroy(e);
        for (void* p : allocs) (void)hipFree(p);
    }
    void mark(int stage, bool end, hipStream_t st) {
        if (!profiling) return;
        (void)hipEventRecord(ev[2 * stage + (end ? 1 : 0)], st);
        if (end) ran[stage] = true;
    }
};

namespace {

int check_layer(const llmoe_layer* L) {
    if (!L) return fail(LLMOE_EINVAL, "null layer");
    return LLMOE_OK;
}

int nblocks(const llmoe_layer* L, int T) { return (T + L->d.block - 1) / L->d.block; }

// streamed work items hold 16 slots; the item capacity for T tokens (experts with more than TILED_MIN slots take
// tiled units instead when the routing spans several blocks)
void choose_items(llmoe_layer* L, int T) {
    const auto& d = L->d;
    const long eff = std::min<long>(d.n_experts, long(nblocks(L, T)) * std::min(d.pool, d.n_experts));
    L->ntok = 16;
    const long routed = eff + (long(T) * d.top_k + L->ntok - 1) / L->ntok;
    const long shared = d.has_shared ? (T + L->ntok - 1) / L->ntok : 0;
    L->max_items = int(routed + shared);
    L->tiled = T > d.block && T > TILED_MIN;   // the single-block decode routing emits streamed units only
}

// work-item capacity for T tokens, checked before any kernel of the call is launched: the routing kernels OR
// bits into the layer's token masks and pool maxima, which only the placement kernel clears again
int prepare_items(llmoe_layer* L, int T) {
    choose_items(L, T);
    if (size_t(L->max_items) > L->items_cap)
        return fail(LLMOE_EINVAL, "item capacity exceeded (%d items for T = %d, capacity %zu)", L->max_items, T,
                    L->items_cap);
    return LLMOE_OK;
}

int check_T(const llmoe_layer* L, int T) {
    if (T < 1 || T > L->d.max_tokens) return fail(LLMOE_EINVAL, "T = %d outside [1, max_tokens = %d]", T, L->d.max_tokens);
    return LLMOE_OK;
}

// expert GEMMs of one stage: the streamed units, then (if the routing may have any) the tiled units
hipError_t launch_gemm(int mode, const GemmArgs& g, const GemmArgs& tg, bool tiled, hipStream_t st) {
    // tiled (T > one routing block): every expert's slots are tiled chunks, the streamed lists are empty
    return tiled ? launch_tiled_gemm(mode, tg, st) : launch_expert_gemm(mode, 1, g, 0, st);
}

int plan_and_place(llmoe_layer* L, const int32_t* topk, const float* topw, int T, hipStream_t st) {
    const auto& d = L->d;
    L->mark(LLMOE_STAGE_DISPATCH, false, st);
    HIPCHECK(launch_plan(L->mask, T, d.n_experts, d.top_k, d.block, d.has_shared, L->ntok, L->tiled ? 1 : 0,
                         L->bits_d, L->count, L->start, L->bpre, L->units_gu, L->units_dn, L->tunits_gu,
                         L->tunits_dn, L->n_units, L->g_gu, L->g_dn, L->tstart, int(L->chunks_cap), st));
    HIPCHECK(launch_place(topk, topw, L->mask, L->blockmax, L->bpre, T, d.n_experts, d.top_k, d.block, d.has_shared,
                          L->slot_token, L->slot_weight, L->tok_slots, st));
    L->mark(LLMOE_STAGE_DISPATCH, true, st);
    L->routed_T = T;
    return LLMOE_OK;
}

}  // namespace

namespace {
// Intermediates of llmoe_experts_scratch: one file-scope device array per GPU, sized for LLMOE_SCRATCH_MAX_TOKENS
// tokens of K <= 8 routed slots plus the shared slot. Regions (256-byte aligned): Z fp16 [S, 512], zq int8 [S, 512],
// zs fp32 [S, 4], zsum int32 [S, 4], Y fp32 [S, 2048].
constexpr size_t SCR_S = size_t(LLMOE_SCRATCH_MAX_TOKENS) * 9;
constexpr size_t SCR_Z = 0;
constexpr size_t SCR_ZQ = SCR_Z + SCR_S * 512 * 2;
constexpr size_t SCR_ZS = SCR_ZQ + SCR_S * 512;
constexpr size_t SCR_ZSUM = SCR_ZS + SCR_S * 4 * 4;
constexpr size_t SCR_Y = SCR_ZSUM + SCR_S * 4 * 4;
constexpr size_t SCR_BYTES = SCR_Y + SCR_S * 2048 * 4;
static_assert(SCR_ZQ % 256 == 0 && SCR_ZS % 256 == 0 && SCR_ZSUM % 256 == 0 && SCR_Y % 256 == 0, "alignment");
static_assert(SCR_BYTES == LLMOE_SCRATCH_BYTES, "LLMOE_SCRATCH_BYTES in llmoe.h");

static __device__ __align__(256) uint8_t scratch[SCR_BYTES];

constexpr int SCR_MAX_DEV = 64;
std::mutex g_scr_mu;
uint8_t* g_scr_ptr[SCR_MAX_DEV] = {};   // device address of `scratch` on each GPU (the host symbol is a stand-in)

// the device address of `scratch` on the current GPU, looked up once per GPU by llmoe_layer_create (so that a
// later llmoe_experts_scratch call, possibly under graph capture, makes no runtime lookup)
int scratch_ptr(uint8_t** out) {
    int dev = 0;
    HIPCHECK(hipGetDevice(&dev));
    if (dev < 0 || dev >= SCR_MAX_DEV) return fail(LLMOE_EINVAL, "device %d beyond the scratch table", dev);
    std::lock_guard<std::mutex> lk(g_scr_mu);
    if (!g_scr_ptr[dev]) {
        void* p = nullptr;
        HIPCHECK(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
        if (!p) return fail(LLMOE_EHIP, "hipGetSymbolAddress(scratch) returned NULL");
        g_scr_ptr[dev] = static_cast<uint8_t*>(p);
    }
    *out = g_scr_ptr[dev];
    return LLMOE_OK;
}
}  // namespace

extern "C" {

const char* llmoe_last_error(void) { return g_err.c_str(); }

int llmoe_layer_create(const llmoe_layer_desc* desc, const void* blob, size_t blob_bytes, const uint64_t* gu_off,
                       const uint64_t* d_off, const int8_t* bits, const float* router_w, const float* router_bias,
                       llmoe_layer** out) {
    if (!desc || !blob || !gu_off || !d_off || !bits || !router_bias || !out)
        return fail(LLMOE_EINVAL, "null argument");
    *out = nullptr;
    const llmoe_layer_desc d = *desc;
    if (d.hidden != 2048) return fail(LLMOE_EINVAL, "hidden = %d: this build's GEMM geometry is H = 2048", d.hidden);
    if (d.inter != 512) return fail(LLMOE_EINVAL, "inter = %d: FWHT-512 needs I = 512", d.inter);
    if (d.n_experts < 64 || d.n_experts > 256 || d.n_experts % 64)
        return fail(LLMOE_EINVAL, "n_experts = %d: need 64 <= E <= 256, E %% 64 == 0", d.n_experts);
    if (d.top_k < 1 || d.top_k > 8 || d.top_k > d.n_experts) return fail(LLMOE_EINVAL, "top_k = %d", d.top_k);
    if (d.pool < d.top_k) return fail(LLMOE_EINVAL, "pool = %d < top_k", d.pool);
    if (d.block < 1 || d.block > 32) return fail(LLMOE_EINVAL, "block = %d outside [1, 32]", d.block);
    if (d.max_tokens < 1) return fail(LLMOE_EINVAL, "max_tokens = %d", d.max_tokens);
    const int nexp = d.n_experts + (d.has_shared ? 1 : 0);
    const int H = d.hidden, I = d.inter;
    // validate every matrix against the blob
    std::vector<std::pair<uint64_t, size_t>> mats;
    for (int e = 0; e < nexp; ++e) {
        const int b = bits[e];
        if (tile_wbytes(b) < 0) return fail(LLMOE_EINVAL, "expert %d: bits = %d (need 2, 3, 4 or 8)", e, b);
        const size_t gb = packlib_matrix_bytes(2 * I, H, b), db = packlib_matrix_bytes(H, I, b);
        if (gu_off[e] % 16 || d_off[e] % 16) return fail(LLMOE_EINVAL, "expert %d: offsets must be 16-byte aligned", e);
        if (gu_off[e] + gb > blob_bytes || d_off[e] + db > blob_bytes)
            return fail(LLMOE_EINVAL, "expert %d: matrix beyond the blob (%zu bytes)", e, blob_bytes);
    }
    if (int rc = llmoe::ensure_gemm_setup()) return rc;
    uint8_t* scr = nullptr;
    if (int rc = scratch_ptr(&scr)) return rc;

    llmoe_layer* L = new (std::nothrow) llmoe_layer();
    if (!L) return fail(LLMOE_ENOMEM, "host allocation");
    L->d = d;
    L->nexp = nexp;
    auto bail = [&](int code) {
        delete L;
        return code;
    };
#define ALLOC(ptr, n)                                                                                       \
    do {                                                                                                    \
        if (L->alloc(&(ptr), (n)) != hipSuccess) return bail(fail(LLMOE_ENOMEM, "hipMalloc %s", #ptr));     \
    } while (0)
    // weights: upload the packlib blob to a staging buffer, relayout every distinct matrix into the arena at
    // the same offset (the device layout has the packlib byte count)
    L->arena_bytes = blob_bytes;
    ALLOC(L->arena, blob_bytes);
    uint8_t* staging = nullptr;
    if (hipMalloc(&staging, blob_bytes) != hipSuccess) return bail(fail(LLMOE_ENOMEM, "hipMalloc staging"));
    int rc = LLMOE_OK;
    do {
        hipError_t e = hipMemcpy(staging, blob, blob_bytes, hipMemcpyHostToDevice);
        if (e != hipSuccess) { rc = fail(LLMOE_EHIP, "upload: %s", hipGetErrorString(e)); break; }
        std::set<uint64_t> done;
        for (int x = 0; x < nexp && rc == LLMOE_OK; ++x) {
            const int b = bits[x];
            for (int which = 0; which < 2; ++which) {
                const uint64_t off = which == 0 ? gu_off[x] : d_off[x];
                const int R = which == 0 ? 2 * I : H, K = which == 0 ? H : I;
                if (done.count(off)) continue;   // an aliased entry is laid out once
                done.insert(off);
                L->weight_bytes += packlib_matrix_bytes(R, K, b);
                e = launch_relayout(staging + off, L->arena + off, R, K, b, which == 0, nullptr);
                if (e != hipSuccess) { rc = fail(LLMOE_EHIP, "relayout: %s", hipGetErrorString(e)); break; }
            }
        }
        if (rc != LLMOE_OK) break;
        e = hipDeviceSynchronize();
        if (e != hipSuccess) rc = fail(LLMOE_EHIP, "relayout sync: %s", hipGetErrorString(e));
    } while (0);
    (void)hipFree(staging);
    if (rc != LLMOE_OK) return bail(rc);

    ALLOC(L->gu_off_d, nexp);
    ALLOC(L->d_off_d, nexp);
    ALLOC(L->bits_d, (nexp + 3) & ~3);   // whole dwords: the tiled GEMM reads code widths by scalar dword loads
    ALLOC(L->bias, d.n_experts);
    if (hipMemcpy(L->gu_off_d, gu_off, nexp * sizeof(uint64_t), hipMemcpyHostToDevice) != hipSuccess ||
        hipMemcpy(L->d_off_d, d_off, nexp * sizeof(uint64_t), hipMemcpyHostToDevice) != hipSuccess ||
        hipMemcpy(L->bits_d, bits, nexp, hipMemcpyHostToDevice) != hipSuccess ||
        hipMemcpy(L->bias, router_bias, d.n_experts * sizeof(float), hipMemcpyHostToDevice) != hipSuccess)
        return bail(fail(LLMOE_EHIP, "table upload"));
    if (router_w) {
        ALLOC(L->router_w, size_t(H) * d.n_experts);
        if (hipMemcpy(L->router_w, router_w, size_t(H) * d.n_experts * sizeof(float), hipMemcpyHostToDevice) != hipSuccess)
            return bail(fail(LLMOE_EHIP, "router upload"));
    }
    // workspace
    const size_t Tm = size_t(d.max_tokens), K = size_t(d.top_k), E = size_t(d.n_experts);
    const size_t S = Tm * (K + 1), nbm = (Tm + d.block - 1) / d.block;
    ALLOC(L->xq, Tm * H);
    ALLOC(L->xs, Tm * (H / GROUP));
    ALLOC(L->xsum, Tm * (H / GROUP));
    ALLOC(L->part, size_t(ROUTER_KC) * Tm * E);
    ALLOC(L->topk, Tm * K);
    ALLOC(L->topw, Tm * K);
    ALLOC(L->mask, nbm * E);
    ALLOC(L->bpre, nbm * E);
    ALLOC(L->sig, std::max<size_t>(Tm, size_t(d.block)) * E);
    // token masks and per-block pool maxima are accumulated by atomics: zero here, and left zero again by the
    // kernel that consumes them (place_kernel, dispatch_kernel)
    ALLOC(L->blockmax, nbm * E);
    ALLOC(L->tmask, E);
    ALLOC(L->tcopy, E);

    if (hipMemset(L->blockmax, 0, nbm * E * sizeof(uint32_t)) != hipSuccess ||
        hipMemset(L->mask, 0, nbm * E * sizeof(uint32_t)) != hipSuccess ||
        hipMemset(L->tmask, 0, E * sizeof(uint32_t)) != hipSuccess || 
        hipDeviceSynchronize() != hipSuccess)
        return bail(fail(LLMOE_EHIP, "workspace initialisation"));
    ALLOC(L->count, E);
    ALLOC(L->start, E);
    L->items_cap = E + (Tm * K + 15) / 16 + (Tm + 15) / 16 + 2;
    ALLOC(L->units_gu, L->items_cap * MAX_UNITS_PER_ITEM);
    ALLOC(L->units_dn, L->items_cap * MAX_UNITS_PER_ITEM);
    ALLOC(L->n_units, 4);
    L->chunks_cap = E + (Tm * K + TILED_NTOK - 1) / TILED_NTOK + (Tm + TILED_NTOK - 1) / TILED_NTOK + 2;
    if ((5 * L->chunks_cap + 2) * sizeof(uint32_t) > 65536)
        return bail(fail(LLMOE_EINVAL, "max_tokens = %d: more tiled chunks than the planner holds", int(Tm)));
    ALLOC(L->tunits_gu, L->chunks_cap);
    ALLOC(L->tunits_dn, L->chunks_cap);
    L->g_gu = tiled_grid(GEMM_GATE_UP);
    L->g_dn = tiled_grid(GEMM_DOWN);
    if (L->g_gu < 1 || L->g_dn < 1) return bail(fail(LLMOE_EHIP, "tiled GEMM occupancy query failed"));
    ALLOC(L->tstart, size_t(L->g_gu + L->g_dn + 2));
    ALLOC(L->slot_token, S);
    ALLOC(L->slot_weight, S);
    ALLOC(L->tok_slots, Tm * (K + 1));
    ALLOC(L->Z, S * I);
    ALLOC(L->zq, S * I);
    ALLOC(L->zs, S * (I / GROUP));
    ALLOC(L->zsum, S * (I / GROUP));
    ALLOC(L->Y, S * H);
    ALLOC(L->p_item, MAX_UNITS_PER_ITEM);
    ALLOC(L->p_count, 1);
#undef ALLOC
    *out = L;
    g_err.clear();
    return LLMOE_OK;
}

int llmoe_layer_destroy(llmoe_layer* layer) {
    if (!layer) return LLMOE_OK;
    const hipError_t e = hipDeviceSynchronize();
    delete layer;
    if (e != hipSuccess) return fail(LLMOE_EHIP, "destroy sync: %s", hipGetErrorString(e));
    return LLMOE_OK;
}

int llmoe_quantize_a8(const float* x, int rows, int cols, int8_t* q, float* s, int32_t* sum, llmoe_stream stream) {
    if (!x || !q || !s || !sum) return fail(LLMOE_EINVAL, "null argument");
    if (rows < 0 || cols <= 0 || cols % 512) return fail(LLMOE_EINVAL, "A8 shape %d x %d (cols %% 512 == 0)", rows, cols);
    HIPCHECK(launch_quant_a8(x, rows, cols, q, s, sum, static_cast<hipStream_t>(stream)));
    return LLMOE_OK;
}

}  // extern "C"

namespace {
// routing; with quant set (and x given) the router kernel also writes the A8 of x into the layer workspace; with
// xa8 set (routing from logits) the first per-token routing kernel writes the A8 of xa8 there
int route_impl(llmoe_layer* L, const float* x, const float* logits, int T, hipStream_t st, bool quant,
               const float* xa8 = nullptr, bool defer_dispatch = false) {
    const auto& d = L->d;
    L->routed_T = -1;
    if (L->plan_pending) {   // a forward's routing masks that no expert call consumed
        L->plan_pending = false;
        HIPCHECK(launch_zero_decode_state(L->blockmax, L->tmask, d.n_experts, st));
    }
    if (int rc = prepare_items(L, T)) return rc;
    const float* part = logits;
    int nchunks = 1;
    if (x) {
        if (!L->router_w) return fail(LLMOE_EINVAL, "layer created without a router matrix");
        L->mark(LLMOE_STAGE_ROUTER, false, st);
        HIPCHECK(launch_router_logits(x, L->router_w, T, d.hidden, d.n_experts, L->part, quant ? L->xq : nullptr,
                                      quant ? L->xs : nullptr, quant ? L->xsum : nullptr, st));
        L->mark(LLMOE_STAGE_ROUTER, true, st);
        part = L->part;
        nchunks = ROUTER_KC;
    }
    const QuantX qx{x ? nullptr : xa8, L->xq, L->xs, L->xsum};
    L->mark(LLMOE_STAGE_ROUTE, false, st);
    if (T <= d.block) {   // one routing block (a decode step): route, plan and place in one workgroup
        HIPCHECK(launch_decode_route(part, nchunks, L->bias, T, d.n_experts, d.top_k, d.pool, d.routed_scale, L->sig,
                                     L->topk, L->topw, L->blockmax, L->tmask, d.has_shared, L->bits_d,
                                     L->count, L->start, L->units_gu, L->units_dn, L->n_units, L->slot_token,
                                     L->slot_weight, L->tok_slots, qx, defer_dispatch ? 0 : 1, st));
        L->mark(LLMOE_STAGE_ROUTE, true, st);
        L->routed_T = T;
        L->plan_pending = defer_dispatch;
        return LLMOE_OK;
    }
    HIPCHECK(launch_route(part, nchunks, L->bias, T, d.n_experts, d.top_k, d.pool, d.block, d.routed_scale, L->sig,
                          L->blockmax, L->topk, L->topw, L->mask, qx, st));
    L->mark(LLMOE_STAGE_ROUTE, true, st);
    return plan_and_place(L, L->topk, L->topw, T, st);
}
}  // namespace

extern "C" {

int llmoe_route(llmoe_layer* L, const float* x, const float* logits, int T, llmoe_stream stream) {
    if (int rc = check_layer(L)) return rc;
    if (int rc = check_T(L, T)) return rc;
    if ((x == nullptr) == (logits == nullptr)) return fail(LLMOE_EINVAL, "exactly one of x and logits must be given");
    return route_impl(L, x, logits, T, static_cast<hipStream_t>(stream), false);
}

int llmoe_dispatch(llmoe_layer* L, const int32_t* topk, const float* topw, int T, llmoe_stream stream) {
    if (int rc = check_layer(L)) return rc;
    if (int rc = check_T(L, T)) return rc;
    if (!topk || !topw) return fail(LLMOE_EINVAL, "null argument");
    const auto& d = L->d;
    const hipStream_t st = static_cast<hipStream_t>(stream);
    L->routed_T = -1;
    if (L->plan_pending) {   // a forward's routing masks that no expert call consumed
        L->plan_pending = false;
        HIPCHECK(launch_zero_decode_state(L->blockmax, L->tmask, d.n_experts, st));
    }
    if (int rc = prepare_items(L, T)) return rc;
    HIPCHECK(hipMemcpyAsync(L->topk, topk, size_t(T) * d.top_k * sizeof(int32_t), hipMemcpyDeviceToDevice, st));
    HIPCHECK(hipMemcpyAsync(L->topw, topw, size_t(T) * d.top_k * sizeof(float), hipMemcpyDeviceToDevice, st));
    HIPCHECK(launch_masks(L->topk, T, d.n_experts, d.top_k, d.block, L->mask, st));
    return plan_and_place(L, L->topk, L->topw, T, st);
}

}  // extern "C"

namespace {
Inter layer_inter(const llmoe_layer* L) { return Inter{L->Z, L->zq, L->zs, L->zsum, L->Y}; }

int experts_impl(llmoe_layer* L, const int8_t* xq, const float* xs, const int32_t* xsum, int T, float* out,
                 const NormOut& no, const Inter& w, hipStream_t st) {
    if (T != L->routed_T) return fail(LLMOE_ESTATE, "no routing for T = %d (route or dispatch first)", T);
    const auto& d = L->d;
    const int H = d.hidden, I = d.inter, K = d.top_k;
    const int S = T * K + (d.has_shared ? T : 0);
    GemmArgs g{};
    g.base = L->arena;
    g.bits = L->bits_d;
    g.slot_weight = L->slot_weight;
    // gate_up: B rows are token rows of x'
    g.items = L->units_gu;
    g.n_items = L->n_units;
    g.off = L->gu_off_d;
    g.slot_token = L->slot_token;
    g.xq = xq; g.xs = xs; g.xsum = xsum;
    g.K = H; g.R = 2 * I; g.Z = w.Z;
    g.fast = L->fast ? 1 : 0;
    GemmArgs tg = g;
    tg.items = L->tunits_gu;
    tg.tstart = L->tstart;
    tg.n_items = L->n_units + 2;
    L->last_gu = g;
    L->last_tgu = tg;
    // a forward's decode step: the gate_up GEMM builds the slot plan from the routing masks and writes the lists
    // that the dispatch kernel would have (re-launches for stage timing then read those lists)
    const bool plan = L->plan_pending && !L->tiled;
    L->plan_pending = false;
    L->last_plan = plan;
    L->mark(LLMOE_STAGE_GATE_UP, false, st);
    if (plan) {
        const DecodePlanArgs pa{T, d.n_experts, K, L->tmask, L->tcopy, L->topk, L->topw,
                                DispatchOut{d.has_shared, 16, L->bits_d, L->count, L->start, L->units_gu, L->units_dn,
                                            L->n_units, L->slot_token, L->slot_weight, L->tok_slots},
                                L->d_off_d, DOWN_PF_BYTES};
        L->last_pa = pa;
        L->last_pa.tmask = L->tcopy;   // a re-launch plans from the copy
        HIPCHECK(launch_expert_gemm_plan(g, pa, st));
    } else {
        HIPCHECK(launch_gemm(GEMM_GATE_UP, g, tg, L->tiled, st));
    }
    L->mark(LLMOE_STAGE_GATE_UP, true, st);
    L->mark(LLMOE_STAGE_FWHT, false, st);
    // FWHT-512 + A8 of Z: its own kernel before the tiled down GEMM; the streamed down GEMM stages it per item
    // (measured in the tiled down GEMM's chunk staging too: 81 -> 96 us per config-3 layer against a 10.6 us kernel)
    if (L->tiled) HIPCHECK(launch_fwht_a8(w.Z, S, w.zq, w.zs, w.zsum, st));
    L->mark(LLMOE_STAGE_FWHT, true, st);
    // down: B rows are slot rows of Z'
    g.items = L->units_dn;
    g.n_items = L->n_units + 1;
    g.off = L->d_off_d;
    g.slot_token = nullptr;
    g.xq = w.zq; g.xs = w.zs; g.xsum = w.zsum;
    g.K = I; g.R = H; g.Z = nullptr; g.Y = w.Y;
    // fast numerics with several routing blocks: the slot outputs are rounded to fp16 (half the bytes through HBM
    // for Y and the combine). A decode step's Y stays in the caches, where fp32 costs nothing more.
    const bool yhalf = L->fast && L->tiled;
    g.Yh = yhalf ? reinterpret_cast<uint16_t*>(w.Y) : nullptr;
    g.fast = 0;
    tg = g;
    g.zin = w.Z; g.xq_out = w.zq; g.xs_out = w.zs; g.xsum_out = w.zsum;
    if (plan) {
        g.clear_a = L->tmask;
        g.clear_b = L->blockmax;
        g.nclear = d.n_experts;
    }
    tg.items = L->tunits_dn;
    tg.tstart = L->tstart + L->g_gu + 1;
    tg.n_items = L->n_units + 3;
    L->last_dn = g;
    L->last_tdn = tg;
    L->last_S = S; L->last_T = T; L->last_tiled = L->tiled; L->last_out = out; L->last_norm = no; L->last_w = w;
    L->last_yhalf = yhalf;
    L->have_last = true;
    L->mark(LLMOE_STAGE_DOWN, false, st);
    HIPCHECK(launch_gemm(GEMM_DOWN, g, tg, L->tiled, st));
    L->mark(LLMOE_STAGE_DOWN, true, st);
    L->mark(LLMOE_STAGE_COMBINE, false, st);
    if (no.h)
        HIPCHECK(launch_combine_norm(w.Y, yhalf, L->tok_slots, T, K + (d.has_shared ? 1 : 0), K + 1, no.signs,
                                     no.eps, no.h, no.q, no.s, no.sum, st));
    else
        HIPCHECK(launch_combine(w.Y, yhalf, L->tok_slots, T, H, K + (d.has_shared ? 1 : 0), K + 1, out, st));
    L->mark(LLMOE_STAGE_COMBINE, true, st);
    return LLMOE_OK;
}
}  // namespace

extern "C" {

int llmoe_experts(llmoe_layer* L, const int8_t* xq, const float* xs, const int32_t* xsum, int T, float* out,
                  llmoe_stream stream) {
    if (int rc = check_layer(L)) return rc;
    if (!xq || !xs || !xsum || !out) return fail(LLMOE_EINVAL, "null argument");
    return experts_impl(L, xq, xs, xsum, T, out, NormOut{}, layer_inter(L), static_cast<hipStream_t>(stream));
}

int llmoe_experts_norm(llmoe_layer* L, const int8_t* xq, const float* xs, const int32_t* xsum, int T,
                       const float* signs, float eps, float* h, int8_t* q_next, float* s_next, int32_t* sum_next,
                       llmoe_stream stream) {
    if (int rc = check_layer(L)) return rc;
    if (!xq || !xs || !xsum || !signs || !h || !q_next || !s_next || !sum_next)
        return fail(LLMOE_EINVAL, "null argument");
    if (L->d.hidden != 2048) return fail(LLMOE_EINVAL, "the rotation is FWHT-2048: hidden must be 2048");
    if (L->d.top_k + (L->d.has_shared ? 1 : 0) > 9) return fail(LLMOE_EINVAL, "at most 9 slots per token");
    return experts_impl(L, xq, xs, xsum, T, nullptr, NormOut{signs, eps, h, q_next, s_next, sum_next},
                        layer_inter(L), static_cast<hipStream_t>(stream));
}

}  // extern "C"


extern "C" {

int llmoe_experts_scratch(llmoe_layer* L, const int8_t* xq, const float* xs, const int32_t* xsum, int T, float* out,
                          llmoe_stream stream) {
    if (int rc = check_layer(L)) return rc;
    if (!xq || !xs || !xsum || !out) return fail(LLMOE_EINVAL, "null argument");
    if (T < 1 || T > LLMOE_SCRATCH_MAX_TOKENS)
        return fail(LLMOE_EINVAL, "T = %d outside [1, %d] (the static scratch of llmoe_experts_scratch)", T,
                    LLMOE_SCRATCH_MAX_TOKENS);
    if (L->d.hidden != 2048 || L->d.inter != 512 || L->d.top_k > 8)
        return fail(LLMOE_EINVAL, "the static scratch is sized for hidden 2048, inter 512, top_k <= 8");
    uint8_t* base = nullptr;
    if (int rc = scratch_ptr(&base)) return rc;
    const Inter w{reinterpret_cast<uint16_t*>(base + SCR_Z), reinterpret_cast<int8_t*>(base + SCR_ZQ),
                  reinterpret_cast<float*>(base + SCR_ZS), reinterpret_cast<int32_t*>(base + SCR_ZSUM),
                  reinterpret_cast<float*>(base + SCR_Y)};
    return experts_impl(L, xq, xs, xsum, T, out, NormOut{}, w, static_cast<hipStream_t>(stream));
}

int llmoe_layer_forward(llmoe_layer* L, const float* x, const float* logits, int T, float* out, llmoe_stream stream) {
    if (int rc = check_layer(L)) return rc;
    if (int rc = check_T(L, T)) return rc;
    if (!x || !out) return fail(LLMOE_EINVAL, "null argument");
    const hipStream_t st = static_cast<hipStream_t>(stream);
    if (!logits && !L->router_w) return fail(LLMOE_EINVAL, "layer created without a router matrix");
    // the A8 of x rides on the first routing kernel: the router's (x·Wr) or, from given logits, the per-token one
    // at decode the dispatch is left to the gate_up GEMM (plan_pending)
    if (int rc = route_impl(L, logits ? nullptr : x, logits, T, st, logits == nullptr, logits ? x : nullptr, true))
        return rc;
    return llmoe_experts(L, L->xq, L->xs, L->xsum, T, out, stream);
}

int llmoe_layer_forward_norm(llmoe_layer* L, const float* x, const float* logits, int T, const float* signs,
                             float eps, float* h, int8_t* q_next, float* s_next, int32_t* sum_next,
                             llmoe_stream stream) {
    if (int rc = check_layer(L)) return rc;
    if (int rc = check_T(L, T)) return rc;
    if (!x || !signs || !h || !q_next || !s_next || !sum_next) return fail(LLMOE_EINVAL, "null argument");
    if (L->d.hidden != 2048) return fail(LLMOE_EINVAL, "the rotation is FWHT-2048: hidden must be 2048");
    if (L->d.top_k + (L->d.has_shared ? 1 : 0) > 9) return fail(LLMOE_EINVAL, "at most 9 slots per token");
    if (!logits && !L->router_w) return fail(LLMOE_EINVAL, "layer created without a router matrix");
    const hipStream_t st = static_cast<hipStream_t>(stream);
    // as llmoe_layer_forward: the A8 of x rides on the first routing kernel, the dispatch on the gate_up GEMM
    if (int rc = route_impl(L, logits ? nullptr : x, logits, T, st, logits == nullptr, logits ? x : nullptr, true))
        return rc;
    return experts_impl(L, L->xq, L->xs, L->xsum, T, nullptr, NormOut{signs, eps, h, q_next, s_next, sum_next},
                        layer_inter(L), st);
}

int llmoe_layer_set_numerics(llmoe_layer* L, int mode) {
    if (int rc = check_layer(L)) return rc;
    if (mode != LLMOE_NUMERICS_EXACT && mode != LLMOE_NUMERICS_FAST) return fail(LLMOE_EINVAL, "numerics mode %d", mode);
    L->fast = mode == LLMOE_NUMERICS_FAST;
    return LLMOE_OK;
}

int llmoe_layer_set_profiling(llmoe_layer* L, int enabled) {
    if (int rc = check_layer(L)) return rc;
    if (enabled) {
        for (hipEvent_t& e : L->ev)
            if (!e) HIPCHECK(hipEventCreate(&e));
        for (bool& r : L->ran) r = false;
    }
    L->profiling = enabled != 0;
    return LLMOE_OK;
}

int llmoe_layer_stage_ms(llmoe_layer* L, float* ms) {
    if (int rc = check_layer(L)) return rc;
    if (!ms) return fail(LLMOE_EINVAL, "null argument");
    for (int i = 0; i < LLMOE_N_STAGES; ++i) {
        ms[i] = -1.0f;
        if (!L->ran[i]) continue;
        HIPCHECK(hipEventSynchronize(L->ev[2 * i + 1]));
        HIPCHECK(hipEventElapsedTime(&ms[i], L->ev[2 * i], L->ev[2 * i + 1]));
    }
    return LLMOE_OK;
}

namespace {
hipError_t relaunch_stage(llmoe_layer* L, int stage, hipStream_t st) {
    const auto& d = L->d;
    switch (stage) {
        case LLMOE_STAGE_GATE_UP:   // the kernel the call ran (a decode forward's plans again, from the copied masks)
            return L->last_plan ? launch_expert_gemm_plan(L->last_gu, L->last_pa, st)
                                : launch_gemm(GEMM_GATE_UP, L->last_gu, L->last_tgu, L->last_tiled, st);
        case LLMOE_STAGE_DOWN: return launch_gemm(GEMM_DOWN, L->last_dn, L->last_tdn, L->last_tiled, st);
        case LLMOE_STAGE_FWHT:
            // one routing block: FWHT-512 + A8 runs inside the streamed down GEMM (its time is in that stage)
            if (!L->last_tiled) return hipErrorNotSupported;
            return launch_fwht_a8(L->last_w.Z, L->last_S, L->last_w.zq, L->last_w.zs, L->last_w.zsum, st);
        case LLMOE_STAGE_COMBINE:
            if (L->last_norm.h)   // re-adds into h: each repeat moves the residual stream on by one more layer
                return launch_combine_norm(L->last_w.Y, L->last_yhalf, L->tok_slots, L->last_T,
                                           d.top_k + (d.has_shared ? 1 : 0), d.top_k + 1, L->last_norm.signs,
                                           L->last_norm.eps, L->last_norm.h, L->last_norm.q, L->last_norm.s,
                                           L->last_norm.sum, st);
            return launch_combine(L->last_w.Y, L->last_yhalf, L->tok_slots, L->last_T, d.hidden,
                                  d.top_k + (d.has_shared ? 1 : 0), d.top_k + 1, L->last_out, st);
        default: return hipErrorInvalidValue;
    }
}
}  // namespace

int llmoe_layers_time_stage(llmoe_layer* const* layers, int n, int stage, int reps, llmoe_stream stream,
                            float* avg_ms) {
    if (!layers || n < 1 || !avg_ms || reps < 1) return fail(LLMOE_EINVAL, "bad argument");
    if (stage != LLMOE_STAGE_GATE_UP && stage != LLMOE_STAGE_DOWN && stage != LLMOE_STAGE_FWHT &&
        stage != LLMOE_STAGE_COMBINE)
        return fail(LLMOE_EINVAL, "stage %d cannot be re-launched", stage);
    for (int i = 0; i < n; ++i) {
        if (int rc = check_layer(layers[i])) return rc;
        if (!layers[i]->have_last) return fail(LLMOE_ESTATE, "layer %d: no llmoe_experts call to repeat", i);
        if (stage == LLMOE_STAGE_FWHT && !layers[i]->last_tiled)
            return fail(LLMOE_ESTATE, "layer %d: at one routing block FWHT-512 + A8 is fused into the down GEMM "
                                      "(time LLMOE_STAGE_DOWN)", i);
    }
    const hipStream_t st = static_cast<hipStream_t>(stream);
    hipEvent_t a, b;
    HIPCHECK(hipEventCreate(&a));
    HIPCHECK(hipEventCreate(&b));
    for (int i = 0; i < n; ++i) HIPCHECK(relaunch_stage(layers[i], stage, st));   // warm
    HIPCHECK(hipEventRecord(a, st));
    for (int r = 0; r < reps; ++r)
        for (int i = 0; i < n; ++i) HIPCHECK(relaunch_stage(layers[i], stage, st));
    HIPCHECK(hipEventRecord(b, st));
    HIPCHECK(hipEventSynchronize(b));
    float ms = 0.0f;
    HIPCHECK(hipEventElapsedTime(&ms, a, b));
    (void)hipEventDestroy(a);
    (void)hipEventDestroy(b);
    *avg_ms = ms / float(reps * n);
    return LLMOE_OK;
}

int llmoe_layer_time_stage(llmoe_layer* L, int stage, int reps, llmoe_stream stream, float* avg_ms) {
    return llmoe_layers_time_stage(&L, 1, stage, reps, stream, avg_ms);
}

int llmoe_layer_buffers(const llmoe_layer* L, llmoe_buffers* o) {
    if (int rc = check_layer(L)) return rc;
    if (!o) return fail(LLMOE_EINVAL, "null argument");
    o->xq = L->xq; o->xs = L->xs; o->xsum = L->xsum;
    o->logits_part = L->part;
    o->topk = L->topk; o->topw = L->topw;
    o->count = L->count; o->start = L->start;
    o->slot_token = L->slot_token; o->slot_weight = L->slot_weight; o->tok_slots = L->tok_slots;
    o->items = reinterpret_cast<int32_t*>(L->units_gu); o->n_items = L->n_units;
    o->Z = L->Z; o->zq = L->zq; o->zs = L->zs; o->zsum = L->zsum; o->Y = L->Y;
    o->ntok = L->ntok; o->max_items = L->max_items;
    return LLMOE_OK;
}

int llmoe_layer_weight_bytes(const llmoe_layer* L, size_t* bytes) {
    if (int rc = check_layer(L)) return rc;
    if (!bytes) return fail(LLMOE_EINVAL, "null argument");
    *bytes = L->weight_bytes;
    return LLMOE_OK;
}

int llmoe_selftest_f16(uint64_t* mismatches) {
    if (!mismatches) return fail(LLMOE_EINVAL, "null argument");
    unsigned long long* d = nullptr;
    HIPCHECK(hipMalloc(&d, sizeof(*d)));
    hipError_t e = hipMemset(d, 0, sizeof(*d));
    if (e == hipSuccess) e = launch_f16_selftest(d, nullptr);
    unsigned long long h = 0;
    if (e == hipSuccess) e = hipMemcpy(&h, d, sizeof(h), hipMemcpyDeviceToHost);
    (void)hipFree(d);
    if (e != hipSuccess) return fail(LLMOE_EHIP, "f16 self-test: %s", hipGetErrorString(e));
    *mismatches = h;
    return LLMOE_OK;
}

int llmoe_group_products(llmoe_layer* L, int expert, int which, const int8_t* xq, const int32_t* xsum, int n,
                         int32_t* P, llmoe_stream stream) {
    if (int rc = check_layer(L)) return rc;
    if (!xq || !xsum || !P) return fail(LLMOE_EINVAL, "null argument");
    if (expert < 0 || expert >= L->nexp) return fail(LLMOE_EINVAL, "expert %d", expert);
    if (which != 0 && which != 1) return fail(LLMOE_EINVAL, "which = %d", which);
    if (n < 1 || n > 64) return fail(LLMOE_EINVAL, "n = %d outside [1, 64]", n);
    const hipStream_t st = static_cast<hipStream_t>(stream);
    int b8 = 0;
    HIPCHECK(hipMemcpy(&b8, L->bits_d + expert, 1, hipMemcpyDeviceToHost));
    const int nrb = gemm_row_blocks(which == 1, int(int8_t(b8)));
    for (int r = 0; r < nrb; ++r) L->p_item_host[r] = Item{expert, 0, n, r};
    L->p_count_host = nrb;
    HIPCHECK(hipMemcpyAsync(L->p_item, L->p_item_host, nrb * sizeof(Item), hipMemcpyHostToDevice, st));
    HIPCHECK(hipMemcpyAsync(L->p_count, &L->p_count_host, sizeof(int), hipMemcpyHostToDevice, st));
    GemmArgs g{};
    g.base = L->arena;
    g.off = which == 0 ? L->gu_off_d : L->d_off_d;
    g.bits = L->bits_d;
    g.items = L->p_item;
    g.n_items = L->p_count;
    g.xq = xq; g.xs = nullptr; g.xsum = xsum;
    g.K = which == 0 ? L->d.hidden : L->d.inter;
    g.R = which == 0 ? 2 * L->d.inter : L->d.hidden;
    g.P = P;
    HIPCHECK(launch_expert_gemm(which == 0 ? GEMM_PRODUCTS_GATE_UP : GEMM_PRODUCTS_DOWN, 4, g, 1, st));
    HIPCHECK(hipStreamSynchronize(st));   // the host item record must outlive the copy
    return LLMOE_OK;
}

}  // extern "C"
