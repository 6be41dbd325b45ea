// Activation kernels of the MoE layer: the A8 quantiser of the layer input, the FWHT-512 + A8 of the down
// input, and the fixed-order weighted combine. One 64-lane wavefront covers 512 values (8 per lane), so a
// 128-group is 16 lanes and every group reduction is 4 butterfly shuffles.
#include "llmoe_internal.h"

namespace llmoe {

namespace {

// A8 of rows of fp32 (engine/ops.cu:42-66): s = max(max|v| / 127, 1e-30), q = clamp(rint(v / s), +-127).
// One wave per 512 columns of one row; grid (cols/512/4 rounded up, rows), 256 threads.
__global__ void __launch_bounds__(256) quant_a8_kernel(const float* __restrict__ x, int rows, int cols,
                                                       int8_t* __restrict__ q, float* __restrict__ s,
                                                       int* __restrict__ sum) {
    const int lane = threadIdx.x & 63;
    const int chunk = blockIdx.x * 4 + (threadIdx.x >> 6), row = blockIdx.y;
    if (chunk * 512 >= cols || row >= rows) return;
    const size_t base = size_t(row) * cols + size_t(chunk) * 512;
    const size_t gi = size_t(row) * (cols / GROUP) + size_t(chunk) * 4;
    quant_a8_512(x + base, lane, q + base, s + gi, sum + gi);
}

// Z' = A8(Z H512 / sqrt(512)) per slot (engine/moe_i8.cu:447-502), one wave per slot (fwht512_a8).
// grid ceil(n/4), 256 threads.
__global__ void __launch_bounds__(256) fwht_a8_kernel(const uint16_t* __restrict__ Z, int nslots,
                                                      int8_t* __restrict__ q, float* __restrict__ s,
                                                      int* __restrict__ sum) {
    const int lane = threadIdx.x & 63;
    const int slot = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (slot >= nslots) return;
    uint2 qw;
    float sc;
    int tot;
    fwht512_a8(Z + size_t(slot) * 512, lane, qw, sc, tot);
    *reinterpret_cast<uint2*>(q + size_t(slot) * 512 + 8 * lane) = qw;
    if ((lane & 15) == 0) {
        s[size_t(slot) * 4 + (lane >> 4)] = sc;
        sum[size_t(slot) * 4 + (lane >> 4)] = tot;
    }
}

// out[t, :] = sum_{k < kk} Y[tok_slots[t, k], :], k ascending (engine/moe_i8.cu:505-515). grid (T, column slices).
constexpr int MAX_KK = 9;   // top-8 + the shared expert
// 4 consecutive slot outputs from element index i of Y: fp32, or fp16 bits (HALF, the fast-numerics down output).
// STREAM: non-temporal loads, for an fp32 Y far larger than the caches (more than 256 tokens: the combine then
// reads 5-8 % faster), not for a decode step's Y, which is still in the caches (there they cost 1.5 us), nor for
// fp16 rows (measured 6-35 % slower).
template <bool HALF, bool STREAM = false>
__device__ __forceinline__ float4 load_y4(const void* __restrict__ Y, size_t i) {
    typedef float v4f __attribute__((ext_vector_type(4)));
    typedef unsigned int v2u __attribute__((ext_vector_type(2)));
    if constexpr (HALF) {
        const v2u* p = reinterpret_cast<const v2u*>(static_cast<const uint16_t*>(Y) + i);
        const v2u u = STREAM ? __builtin_nontemporal_load(p) : *p;
        return make_float4(f16_bits_to_f32(u.x & 0xFFFFu), f16_bits_to_f32(u.x >> 16), f16_bits_to_f32(u.y & 0xFFFFu),
                           f16_bits_to_f32(u.y >> 16));
    } else {
        const v4f* p = reinterpret_cast<const v4f*>(static_cast<const float*>(Y) + i);
        const v4f v = STREAM ? __builtin_nontemporal_load(p) : *p;
        return make_float4(v.x, v.y, v.z, v.w);
    }
}

template <bool HALF, bool STREAM>
__global__ void __launch_bounds__(256) combine_kernel(const void* __restrict__ Y, const int* __restrict__ tok_slots,
                                                      int H, int kk, int K1, float* __restrict__ out) {
    const int t = blockIdx.x;
    // columns [h0, h1) of the row: gridDim.y slices, so that a small T still spreads over many CUs
    const int hw = H / int(gridDim.y), h0 = int(blockIdx.y) * hw, h1 = h0 + hw;
    int sl[MAX_KK];   // (scalar loads: the row's slots are the same for the whole workgroup)
#pragma unroll
    for (int k = 0; k < MAX_KK; ++k) sl[k] = k < kk ? *const_ptr(tok_slots + t * K1 + k) : 0;
    if constexpr (HALF) {
        // fp16 rows: 8 columns (16 bytes of each row) per thread and pass, the same ordered sums
        for (int hb = h0 + threadIdx.x * 8; hb < h1; hb += blockDim.x * 8) {
            uint4 raw[MAX_KK];
#pragma unroll
            for (int k = 0; k < MAX_KK; ++k)
                if (k < kk)
                    raw[k] = *reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(Y) + size_t(sl[k]) * H + hb);
            float acc[8] = {0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int k = 0; k < MAX_KK; ++k) {
                if (k < kk) {
                    const uint32_t w[4] = {raw[k].x, raw[k].y, raw[k].z, raw[k].w};
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        acc[2 * j] = acc[2 * j] + f16_bits_to_f32(w[j] & 0xFFFFu);
                        acc[2 * j + 1] = acc[2 * j + 1] + f16_bits_to_f32(w[j] >> 16);
                    }
                }
            }
            float4* o = reinterpret_cast<float4*>(out + size_t(t) * H + hb);
            o[0] = make_float4(acc[0], acc[1], acc[2], acc[3]);
            o[1] = make_float4(acc[4], acc[5], acc[6], acc[7]);
        }
        return;
    }
    // R float4 columns per thread per pass: every load of the pass is in flight before the ordered sums
    constexpr int R = 2;
    for (int hb = h0 + threadIdx.x * 4; hb < h1; hb += blockDim.x * 4 * R) {
        float4 v[R][MAX_KK];
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const int h = hb + r * blockDim.x * 4;
#pragma unroll
            for (int k = 0; k < MAX_KK; ++k)
                if (k < kk && h < h1) v[r][k] = load_y4<HALF, STREAM>(Y, size_t(sl[k]) * H + h);
        }
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const int h = hb + r * blockDim.x * 4;
            if (h >= h1) break;
            float4 acc = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
#pragma unroll
            for (int k = 0; k < MAX_KK; ++k) {
                if (k < kk) {
                    acc.x = acc.x + v[r][k].x;
                    acc.y = acc.y + v[r][k].y;
                    acc.z = acc.z + v[r][k].z;
                    acc.w = acc.w + v[r][k].w;
                }
            }
            *reinterpret_cast<float4*>(out + size_t(t) * H + h) = acc;
        }
    }
}

// FWHT-2048 of the workgroup's 2048 values, stages h = 1 .. 1024 ascending. On entry thread i holds values
// 8i .. 8i+7 (layout A); bits 0-2 in registers, bits 3-8 by lane shuffles (xor 1 .. 32), then an LDS transpose
// gives thread i the values i + 256 j (layout B) for bits 9-10. On exit x holds layout B.
__device__ __forceinline__ void fwht2048_ab(float (&x)[8], float* v) {
    const int i = threadIdx.x, lane = i & 63;
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
#pragma unroll
    for (int j = 0; j < 8; ++j) v[8 * i + j] = x[j];
    __syncthreads();
#pragma unroll
    for (int j = 0; j < 8; ++j) x[j] = v[i + 256 * j];
#pragma unroll
    for (int h = 2; h < 8; h <<= 1)                       // index bits 9, 10 (j bits 1, 2)
#pragma unroll
        for (int j = 0; j < 8; ++j)
            if (!(j & h)) {
                const float a = x[j], b = x[j + h];
                x[j] = a + b;
                x[j + h] = a - b;
            }
    __syncthreads();                                      // v is reused by the caller
}

// Combine + un-rotation + residual + the next layer's RMSNorm, rotation and A8 (engine/ops.cu:507-549), H = 2048.
// grid T, 256 threads:
//   x = sum_k Y[tok_slots[t, k]] (k ascending); h[t] += (FWHT(x) signs) / sqrt(2048);
//   r = 1 / sqrt(sum h[t]^2 / 2048 + eps); y = FWHT((h[t] r) signs) / sqrt(2048); (q, s, sum) = A8(y)
// Sum of squares: thread i adds h[i + 256 j]^2 for j ascending, a 64-lane xor butterfly, then the 4 wave sums in
// order -- the order the CPU checker uses.
constexpr float INV_SQRT_2048 = 0.02209708691207961f;
template <bool HALF>
__global__ void __launch_bounds__(256) combine_norm_kernel(const void* __restrict__ Y, const int* __restrict__ tok_slots,
                                                           int kk, int K1, const float* __restrict__ signs, float eps,
                                                           float* __restrict__ h, int8_t* __restrict__ q,
                                                           float* __restrict__ s, int* __restrict__ sum) {
    __shared__ __align__(16) float v[2048];
    __shared__ float red[4];
    const int t = blockIdx.x, i = threadIdx.x, lane = i & 63;
    int sl[MAX_KK];
#pragma unroll
    for (int k = 0; k < MAX_KK; ++k) sl[k] = k < kk ? *const_ptr(tok_slots + t * K1 + k) : 0;
    float4 ya[MAX_KK], yb[MAX_KK];
#pragma unroll
    for (int k = 0; k < MAX_KK; ++k)
        if (k < kk) {
            ya[k] = load_y4<HALF>(Y, size_t(sl[k]) * 2048 + 8 * i);
            yb[k] = load_y4<HALF>(Y, size_t(sl[k]) * 2048 + 8 * i + 4);
        }
    float x[8] = {0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int k = 0; k < MAX_KK; ++k)
        if (k < kk) {
            x[0] = x[0] + ya[k].x; x[1] = x[1] + ya[k].y; x[2] = x[2] + ya[k].z; x[3] = x[3] + ya[k].w;
            x[4] = x[4] + yb[k].x; x[5] = x[5] + yb[k].y; x[6] = x[6] + yb[k].z; x[7] = x[7] + yb[k].w;
        }
    fwht2048_ab(x, v);
    float* hr = h + size_t(t) * 2048;
    float sg[8];
    float p = 0.0f;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        const int c = i + 256 * j;
        sg[j] = signs[c];
        x[j] = hr[c] + (x[j] * sg[j]) * INV_SQRT_2048;
        hr[c] = x[j];
        p = p + x[j] * x[j];
    }
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) p = p + xor_lane(p, o);
    if (lane == 0) red[i >> 6] = p;
    __syncthreads();
    const float tot = ((red[0] + red[1]) + red[2]) + red[3];
    const float r = 1.0f / sqrtf(tot / 2048.0f + eps);
#pragma unroll
    for (int j = 0; j < 8; ++j) v[i + 256 * j] = (x[j] * r) * sg[j];
    __syncthreads();
#pragma unroll
    for (int j = 0; j < 8; ++j) x[j] = v[8 * i + j];
    __syncthreads();
    fwht2048_ab(x, v);
#pragma unroll
    for (int j = 0; j < 8; ++j) v[i + 256 * j] = x[j] * INV_SQRT_2048;
    __syncthreads();
    // A8 per 128-group: wave w takes columns 512 w .. 512 w + 511, 16 lanes per group (as quant_a8_kernel)
    const float* vv = v + 512 * (i >> 6) + 8 * lane;
    float m = 0.0f;
    float val[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        val[j] = vv[j];
        m = fmaxf(m, fabsf(val[j]));
    }
    m = group16_max(m);
    const float sc = fmaxf(m / 127.0f, 1e-30f);
    int totq = 0;
    uint32_t w0 = 0, w1 = 0;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        const int qq = clamp127(__builtin_rintf(val[j] / sc));
        totq += qq;
        if (j < 4) w0 |= uint32_t(qq & 0xFF) << (8 * j);
        else w1 |= uint32_t(qq & 0xFF) << (8 * (j - 4));
    }
    *reinterpret_cast<uint2*>(q + size_t(t) * 2048 + 512 * (i >> 6) + 8 * lane) = make_uint2(w0, w1);
    totq = group16_sum(totq);
    if ((lane & 15) == 0) {
        const size_t gi = size_t(t) * 16 + 4 * (i >> 6) + (lane >> 4);
        s[gi] = sc;
        sum[gi] = totq;
    }
}

}  // namespace

// f32_to_f16_rne against f32_to_f16_bits on fp32 bit patterns [start, start + n) (NaN patterns skipped): the
// number of inputs on which they differ is added to *mismatches.
__global__ void __launch_bounds__(256) f16_selftest_kernel(uint32_t start, uint32_t n,
                                                           unsigned long long* __restrict__ mismatches) {
    unsigned int bad = 0;
    for (uint32_t i = blockIdx.x * 256u + threadIdx.x; i < n; i += gridDim.x * 256u) {
        const uint32_t b = start + i;
        if ((b & 0x7fffffffu) > 0x7f800000u) continue;
        const float f = __uint_as_float(b);
        bad += f32_to_f16_rne(f) != f32_to_f16_bits(f) ? 1u : 0u;
    }
    if (bad) atomicAdd(mismatches, (unsigned long long)bad);
}

hipError_t launch_f16_selftest(unsigned long long* mismatches, hipStream_t st) {
    for (uint32_t sign = 0; sign < 2; ++sign) {
        f16_selftest_kernel<<<8192, 256, 0, st>>>(sign << 31, 0x7f800001u, mismatches);
        const hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}

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

hipError_t launch_combine_norm(const void* Y, int yhalf, const int* tok_slots, int T, int kk, int K1,
                               const float* signs, float eps, float* h, int8_t* q, float* s, int* sum, hipStream_t st) {
    if (T <= 0) return hipSuccess;
    if (kk > MAX_KK) return hipErrorInvalidValue;
    if (yhalf) combine_norm_kernel<true><<<T, 256, 0, st>>>(Y, tok_slots, kk, K1, signs, eps, h, q, s, sum);
    else combine_norm_kernel<false><<<T, 256, 0, st>>>(Y, tok_slots, kk, K1, signs, eps, h, q, s, sum);
    return hipGetLastError();
}

hipError_t launch_combine(const void* Y, int yhalf, const int* tok_slots, int T, int H, int kk, int K1, float* out,
                          hipStream_t st) {
    if (T <= 0) return hipSuccess;
    // a decode step's few rows are split over 8 column slices (256 columns, one pass of 64 threads x 2 float4)
    const int ns = T <= 256 && H % 256 == 0 ? H / 256 : 1;
    const dim3 grid(T, ns);
    if (ns > 1) {
        if (yhalf) combine_kernel<true, false><<<grid, 64, 0, st>>>(Y, tok_slots, H, kk, K1, out);
        else combine_kernel<false, false><<<grid, 64, 0, st>>>(Y, tok_slots, H, kk, K1, out);
    } else {   // more than 256 tokens: an fp32 Y (>= 18 MB) streams through (fp16 rows measured slower that way)
        if (yhalf) combine_kernel<true, false><<<grid, 256, 0, st>>>(Y, tok_slots, H, kk, K1, out);
        else combine_kernel<false, true><<<grid, 256, 0, st>>>(Y, tok_slots, H, kk, K1, out);
    }
    return hipGetLastError();
}

}  // namespace llmoe
