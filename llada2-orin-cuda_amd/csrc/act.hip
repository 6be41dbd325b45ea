// Activation kernels of the MoE layer: the A8 quantiser of the layer input, the FWHT-512 + A8 of the down
// input, and the fixed-order weighted combine. One 64-lane wavefront covers 512 values (8 per lane), so a
// 128-group is 16 lanes and every group reduction is 4 butterfly shuffles.
#include "llmoe_internal.h"

namespace llmoe {

namespace {

__device__ __forceinline__ float group16_max(float m) {
#pragma unroll
    for (int o = 1; o < 16; o <<= 1) m = fmaxf(m, __shfl_xor(m, o));
    return m;
}
__device__ __forceinline__ int group16_sum(int v) {
#pragma unroll
    for (int o = 1; o < 16; o <<= 1) v += __shfl_xor(v, o);
    return v;
}
__device__ __forceinline__ int clamp127(float r) { return int(fminf(fmaxf(r, -127.0f), 127.0f)); }

// A8 of rows of fp32 (engine/ops.cu:42-66): s = max(max|v| / 127, 1e-30), q = clamp(rint(v / s), +-127).
// One wave per 512 columns of one row; grid (cols/512/4 rounded up, rows), 256 threads.
__global__ void __launch_bounds__(256) quant_a8_kernel(const float* __restrict__ x, int rows, int cols,
                                                       int8_t* __restrict__ q, float* __restrict__ s,
                                                       int* __restrict__ sum) {
    const int lane = threadIdx.x & 63;
    const int chunk = blockIdx.x * 4 + (threadIdx.x >> 6), row = blockIdx.y;
    if (chunk * 512 >= cols || row >= rows) return;
    const size_t base = size_t(row) * cols + size_t(chunk) * 512 + 8 * lane;
    const float4 a = *reinterpret_cast<const float4*>(x + base);
    const float4 b = *reinterpret_cast<const float4*>(x + base + 4);
    const float v[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
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
    *reinterpret_cast<uint2*>(q + base) = make_uint2(w0, w1);
    tot = group16_sum(tot);
    if ((lane & 15) == 0) {
        const size_t gi = size_t(row) * (cols / GROUP) + size_t(chunk) * 4 + (lane >> 4);
        s[gi] = sc;
        sum[gi] = tot;
    }
}

// Z' = A8(Z H512 / sqrt(512)) per slot (engine/moe_i8.cu:447-502). One wave per slot, lane l owns values
// 8l .. 8l+7: butterfly stages h = 1, 2, 4 in registers, h = 8 .. 256 by lane shuffles (xor 1 .. 32), in
// ascending h. The group quantiser multiplies by 1/s. Logical order out. grid ceil(n/4), 256 threads.
__global__ void __launch_bounds__(256) fwht_a8_kernel(const uint16_t* __restrict__ Z, int nslots,
                                                      int8_t* __restrict__ q, float* __restrict__ s,
                                                      int* __restrict__ sum) {
    const int lane = threadIdx.x & 63;
    const int slot = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (slot >= nslots) return;
    const uint4 raw = *reinterpret_cast<const uint4*>(Z + size_t(slot) * 512 + 8 * lane);
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
        const bool hi = lane & o;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const float y = __shfl_xor(x[j], o);
            x[j] = hi ? y - x[j] : x[j] + y;
        }
    }
    float m = 0.0f;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        x[j] = x[j] * 0.04419417382415922f;
        m = fmaxf(m, fabsf(x[j]));
    }
    m = group16_max(m);
    const float sc = fmaxf(m / 127.0f, 1e-30f), inv = 1.0f / sc;
    int tot = 0;
    uint32_t w0 = 0, w1 = 0;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        const int qq = clamp127(__builtin_rintf(x[j] * inv));
        tot += qq;
        if (j < 4) w0 |= uint32_t(qq & 0xFF) << (8 * j);
        else w1 |= uint32_t(qq & 0xFF) << (8 * (j - 4));
    }
    *reinterpret_cast<uint2*>(q + size_t(slot) * 512 + 8 * lane) = make_uint2(w0, w1);
    tot = group16_sum(tot);
    if ((lane & 15) == 0) {
        s[size_t(slot) * 4 + (lane >> 4)] = sc;
        sum[size_t(slot) * 4 + (lane >> 4)] = tot;
    }
}

// out[t, :] = sum_{k < kk} Y[tok_slots[t, k], :], k ascending (engine/moe_i8.cu:505-515). grid T, 256 threads.
constexpr int MAX_KK = 9;   // top-8 + the shared expert
__global__ void __launch_bounds__(256) combine_kernel(const float* __restrict__ Y, const int* __restrict__ tok_slots,
                                                      int H, int kk, int K1, float* __restrict__ out) {
    const int t = blockIdx.x;
    int sl[MAX_KK];
#pragma unroll
    for (int k = 0; k < MAX_KK; ++k) sl[k] = k < kk ? tok_slots[t * K1 + k] : 0;
    for (int h = threadIdx.x * 4; h < H; h += blockDim.x * 4) {
        float4 v[MAX_KK];
#pragma unroll
        for (int k = 0; k < MAX_KK; ++k)   // every load in flight before the ordered sum
            if (k < kk) v[k] = *reinterpret_cast<const float4*>(Y + size_t(sl[k]) * H + h);
        float4 acc = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
#pragma unroll
        for (int k = 0; k < MAX_KK; ++k) {
            if (k < kk) {
                acc.x = acc.x + v[k].x;
                acc.y = acc.y + v[k].y;
                acc.z = acc.z + v[k].z;
                acc.w = acc.w + v[k].w;
            }
        }
        *reinterpret_cast<float4*>(out + size_t(t) * H + h) = acc;
    }
}

}  // namespace

hipError_t launch_quant_a8(const float* x, int rows, int cols, int8_t* q, float* s, int* sum, hipStream_t st) {
    if (rows <= 0) return hipSuccess;
    const dim3 grid((cols / 512 + 3) / 4, rows);
    quant_a8_kernel<<<grid, 256, 0, st>>>(x, rows, cols, q, s, sum);
    return hipGetLastError();
}

hipError_t launch_fwht_a8(const uint16_t* Z, int nslots, int8_t* q, float* s, int* sum, hipStream_t st) {
    if (nslots <= 0) return hipSuccess;
    fwht_a8_kernel<<<(nslots + 3) / 4, 256, 0, st>>>(Z, nslots, q, s, sum);
    return hipGetLastError();
}

hipError_t launch_combine(const float* Y, const int* tok_slots, int T, int H, int kk, int K1, float* out,
                          hipStream_t st) {
    if (T <= 0) return hipSuccess;
    combine_kernel<<<T, 256, 0, st>>>(Y, tok_slots, H, kk, K1, out);
    return hipGetLastError();
}

}  // namespace llmoe
