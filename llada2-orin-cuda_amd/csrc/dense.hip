// Dense W.A8 projections (engine/engine.cu:380-383, :425, :434: the reference runs qkv, the attention output and
// the lm_head through the expert GEMM as one "expert" holding every token). One [R, 2048] matrix of b-bit codes
// in packlib "i8", relaid out once for the MFMA kernels; a call multiplies T tokens' A8 rows by it:
//     Y[t, r] (=|+=) sum_g fma chain of scale_w[r, g] scale_x[t, g] P_g[r, t]      (the expert GEMMs' epilogue)
// T <= 32: the streamed kernel over items of 16 tokens x row blocks; T > 32: the tiled kernel over chunks of
// <= 64 tokens, the (chunk, row block) tasks split evenly over its resident workgroups.
#include <cstdarg>
#include <cstdio>
#include <new>
#include <vector>

#include "llmoe.h"
#include "llmoe_internal.h"

using namespace llmoe;

struct llmoe_dense {
    int R = 0, K = 0, bits = 0, max_tokens = 0, G = 0;
    uint8_t* arena = nullptr;      // relaid-out matrix
    uint64_t* off = nullptr;       // [1] = 0 (the GEMMs' per-expert matrix offsets)
    int8_t* bits_d = nullptr;      // [1]
    Item* units = nullptr;         // streamed units or tiled chunks of the latest call
    int* n_units = nullptr;        // [1]
    int* tstart = nullptr;         // [G + 1] tiled work partition
    std::vector<void*> allocs;
    ~llmoe_dense() {
        for (void* p : allocs) (void)hipFree(p);
    }
};

namespace {

int dfail(int code, const char* fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof(buf), fmt, ap);
    va_end(ap);
    return set_error(code, buf);
}

#define DHIP(expr)                                                                                         \
    do {                                                                                                   \
        const hipError_t e_ = (expr);                                                                      \
        if (e_ != hipSuccess) return dfail(LLMOE_EHIP, "%s: %s", #expr, hipGetErrorString(e_));           \
    } while (0)

// Work list of a tiled call (T > 32), one workgroup: chunks {0, j per, n, 0} and the partition of the nch nrb equal
// (chunk, row block) tasks: workgroup w starts at task ceil(w N / G) (chunk | rb << TASK_RB_SHIFT).
__global__ void __launch_bounds__(256) dense_plan_kernel(int T, int R, int bits, int G, Item* __restrict__ units,
                                                         int* __restrict__ n_units, int* __restrict__ tstart) {
    const int nch = tiled_chunks(T), per = tiled_per(T), nrb = R / (16 * tiled_waves(false) * tiled_spw(false, bits));
    for (int j = threadIdx.x; j < nch; j += blockDim.x) units[j] = Item{0, j * per, min(per, T - j * per), 0};
    const long long N = (long long)nch * nrb;
    for (int w = threadIdx.x; w <= G; w += blockDim.x) {
        const long long t = ((long long)w * N + G - 1) / G;
        tstart[w] = int(t / nrb) | (int(t % nrb) << TASK_RB_SHIFT);
    }
    if (threadIdx.x == 0) n_units[0] = nch;
}

}  // namespace

extern "C" {

int llmoe_dense_create(int rows, int k, int bits, const uint8_t* blob, size_t blob_bytes, int max_tokens,
                       llmoe_dense** out) {
    if (!out || !blob) return dfail(LLMOE_EINVAL, "null argument");
    *out = nullptr;
    if (k != 2048) return dfail(LLMOE_EINVAL, "k = %d: dense projections take K = 2048", k);
    if (tile_wbytes(bits) < 0) return dfail(LLMOE_EINVAL, "bits = %d (need 2, 3, 4 or 8)", bits);
    if (rows < 256 || rows % 256) return dfail(LLMOE_EINVAL, "rows = %d: need a positive multiple of 256", rows);
    if (max_tokens < 1) return dfail(LLMOE_EINVAL, "max_tokens = %d", max_tokens);
    const size_t bytes = packlib_matrix_bytes(rows, k, bits);
    if (blob_bytes < bytes) return dfail(LLMOE_EINVAL, "blob of %zu bytes, the matrix needs %zu", blob_bytes, bytes);
    if (int rc = ensure_gemm_setup()) return rc;
    llmoe_dense* D = new (std::nothrow) llmoe_dense();
    if (!D) return dfail(LLMOE_ENOMEM, "host allocation");
    D->R = rows;
    D->K = k;
    D->bits = bits;
    D->max_tokens = max_tokens;
    D->G = tiled_grid(GEMM_DENSE);
    auto alloc = [&](void** p, size_t n) {
        if (hipMalloc(p, std::max<size_t>(n, 16)) != hipSuccess) return false;
        D->allocs.push_back(*p);
        return true;
    };
    uint8_t* staging = nullptr;
    const size_t cap = size_t(tiled_chunks(max_tokens));
    bool ok = D->G > 0 && alloc(reinterpret_cast<void**>(&D->arena), bytes) &&
              alloc(reinterpret_cast<void**>(&D->off), sizeof(uint64_t)) &&
              alloc(reinterpret_cast<void**>(&D->bits_d), 4) &&   // a whole dword: read by scalar dword loads
              alloc(reinterpret_cast<void**>(&D->units), cap * sizeof(Item)) &&
              alloc(reinterpret_cast<void**>(&D->n_units), sizeof(int)) &&
              alloc(reinterpret_cast<void**>(&D->tstart), size_t(D->G + 1) * sizeof(int));
    if (!ok) {
        delete D;
        return dfail(LLMOE_ENOMEM, "device allocation");
    }
    const uint64_t zero = 0;
    const int8_t b8 = int8_t(bits);
    hipError_t e = hipMalloc(&staging, bytes);
    if (e == hipSuccess) e = hipMemcpy(staging, blob, bytes, hipMemcpyHostToDevice);
    if (e == hipSuccess) e = launch_relayout(staging, D->arena, rows, k, bits, 0, nullptr);
    if (e == hipSuccess) e = hipMemcpy(D->off, &zero, sizeof(zero), hipMemcpyHostToDevice);
    if (e == hipSuccess) e = hipMemcpy(D->bits_d, &b8, 1, hipMemcpyHostToDevice);
    if (e == hipSuccess) e = hipDeviceSynchronize();
    if (staging) (void)hipFree(staging);
    if (e != hipSuccess) {
        delete D;
        return dfail(LLMOE_EHIP, "dense weights: %s", hipGetErrorString(e));
    }
    *out = D;
    return LLMOE_OK;
}

int llmoe_dense_destroy(llmoe_dense* D) {
    delete D;
    return LLMOE_OK;
}

int llmoe_dense_forward(llmoe_dense* D, const int8_t* xq, const float* xs, const int32_t* xsum, int T, float* y,
                        int accumulate, llmoe_stream stream) {
    if (!D) return dfail(LLMOE_EINVAL, "null dense");
    if (!xq || !xs || !xsum || !y) return dfail(LLMOE_EINVAL, "null argument");
    if (T < 1 || T > D->max_tokens) return dfail(LLMOE_EINVAL, "T = %d outside [1, max_tokens = %d]", T, D->max_tokens);
    const hipStream_t st = static_cast<hipStream_t>(stream);
    const bool tiled = T > 32;
    if (tiled) {   // (T <= 32: the split-K kernel needs no work list)
        dense_plan_kernel<<<1, 256, 0, st>>>(T, D->R, D->bits, D->G, D->units, D->n_units, D->tstart);
        DHIP(hipGetLastError());
    }
    GemmArgs g{};
    g.base = D->arena;
    g.off = D->off;
    g.bits = D->bits_d;
    g.items = D->units;
    g.n_items = D->n_units;
    g.slot_token = nullptr;
    g.xq = xq;
    g.xs = xs;
    g.xsum = xsum;
    g.K = D->K;
    g.R = D->R;
    g.Y = y;
    g.tstart = D->tstart;
    g.accumulate = accumulate ? 1 : 0;
    g.dense_T = T;
    DHIP(tiled ? launch_tiled_gemm(GEMM_DENSE, g, st) : launch_dense_splitk(D->bits, g, st));
    return LLMOE_OK;
}

}  // extern "C"
