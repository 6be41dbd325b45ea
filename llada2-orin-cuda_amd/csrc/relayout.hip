// Load-time conversion of packlib format-"i8" matrices (quant/packlib.py:140-197) into the device layout the
// expert GEMM streams (llmoe_internal.h). Plays the role of the reference's relayout_strips
// (engine/moe_i8.cu:93-121): there the tile bytes are regrouped for NVIDIA m16n8k32 A fragments; here every code
// is moved to the byte the v_mfma_i32_16x16x64_i8 A operand wants, and each bit width is packed so that one
// shift + one mask (2/4-bit) yields a whole operand register.
#include "llmoe_internal.h"

namespace llmoe {

namespace {

// packlib tile geometry: lane pl (0..31), k32-step j, register r, byte b -> (row, col) inside the 16x128 tile
__device__ __forceinline__ int pl_row(int pl, int r) { return (pl >> 2) + 8 * (r & 1); }
__device__ __forceinline__ int pl_col(int pl, int j, int r, int b) { return 32 * j + 16 * (r >> 1) + 4 * (pl & 3) + b; }

// device strip row of packlib strip row p (gate_up interleave: per lane quad q rows gate 2q, up 2q, gate 2q+1,
// up 2q+1; packlib strip rows are gate 0..7 then up 0..7, quant/packlib.py:98-102)
__device__ __forceinline__ int dev_row(int p, int gate_up) {
    if (!gate_up) return p;
    const int j = p & 7, up = p >> 3;
    return 4 * (j >> 1) + 2 * (j & 1) + up;
}

__device__ __forceinline__ int pl_tile_wbytes(int bits) {
    return bits == 8 ? 2048 : bits == 4 ? 1024 : bits == 3 ? 768 : 512;
}

// grid: strips (grid-stride), 256 threads; dynamic LDS 16 K (codes) + 16 (K/128) * 3 (scales, zeros)
__global__ void __launch_bounds__(256) relayout_kernel(const uint8_t* __restrict__ src, uint8_t* __restrict__ dst,
                                                       int nstrips, int K, int bits, int gate_up) {
    extern __shared__ __align__(16) uint8_t lds[];
    const int NT = K / GROUP, NSB = K / SB_K;
    const int WB = pl_tile_wbytes(bits), TB = WB + 48;
    uint8_t* codes = lds;                                                      // [16][K]
    uint16_t* sc = reinterpret_cast<uint16_t*>(lds + 16 * K);                  // [16][NT]
    uint8_t* zr = lds + 16 * K + 32 * NT;                                      // [16][NT]
    const size_t out_sb = sb_bytes(bits);
    for (int s = blockIdx.x; s < nstrips; s += gridDim.x) {
        const uint8_t* tiles = src + size_t(s) * NT * TB;
        // phase 1: packlib tiles -> LDS codes[dev row][col]
        for (int w = threadIdx.x; w < NT * 32; w += blockDim.x) {
            const int tt = w >> 5, pl = w & 31;
            const uint8_t* tile = tiles + size_t(tt) * TB;
            for (int j = 0; j < 4; ++j)
                for (int r = 0; r < 4; ++r)
                    for (int b = 0; b < 4; ++b) {
                        uint32_t v;
                        if (bits == 8) {
                            v = tile[((j * 32 + pl) * 4 + r) * 4 + b];
                        } else if (bits == 4) {
                            const int wd = 2 * j + (r >> 1), u = wd >> 2;
                            v = (tile[((u * 32 + pl) * 4 + (wd & 3)) * 4 + b] >> (4 * (r & 1))) & 0xFu;
                        } else {
                            v = (tile[(pl * 4 + j) * 4 + b] >> (2 * r)) & 3u;
                            if (bits == 3)
                                v |= ((uint32_t(tile[512 + (pl * 2 + (j >> 1)) * 4 + b]) >> (4 * (j & 1) + r)) & 1u) << 2;
                        }
                        codes[dev_row(pl_row(pl, r), gate_up) * K + tt * GROUP + pl_col(pl, j, r, b)] = uint8_t(v);
                    }
        }
        for (int w = threadIdx.x; w < NT * 16; w += blockDim.x) {
            const int tt = w >> 4, p = w & 15;
            const uint8_t* meta = tiles + size_t(tt) * TB + WB;
            const int d = dev_row(p, gate_up);
            sc[d * NT + tt] = uint16_t(meta[2 * p] | (meta[2 * p + 1] << 8));
            zr[d * NT + tt] = meta[32 + p];
        }
        __syncthreads();
        // phase 2: device superblocks
        uint8_t* out = dst + size_t(s) * NSB * out_sb;
        for (int w = threadIdx.x; w < NSB * bits * 64; w += blockDim.x) {
            const int sb = w / (bits * 64), i = (w / 64) % bits, L = w & 63;
            const int q = L >> 4, row = L & 15;
            const uint8_t* cr = codes + row * K + sb * SB_K;
            // code ci (0..31) of tile tau for this lane
            auto code = [&](int tau, int ci) -> uint32_t {
                const int col = 128 * tau + (ci < 16 ? 16 * q + ci : 64 + 16 * q + ci - 16);
                return cr[col];
            };
            uint32_t wd[4];
            for (int m = 0; m < 4; ++m) {
                uint32_t v = 0;
                if (bits == 2 || (bits == 3 && i < 2)) {
                    const int tau = 2 * i + (m >> 1), mm = m & 1;
                    for (int e = 0; e < 4; ++e)
                        for (int sh = 0; sh < 4; ++sh) v |= (code(tau, 4 * (4 * mm + sh) + e) & 3u) << (8 * e + 2 * sh);
                } else if (bits == 3) {
                    const int tau = m;
                    for (int e = 0; e < 4; ++e)
                        for (int sh = 0; sh < 8; ++sh) v |= ((code(tau, 4 * sh + e) >> 2) & 1u) << (8 * e + sh);
                } else if (bits == 4) {
                    const int tau = i;
                    for (int e = 0; e < 4; ++e)
                        v |= ((code(tau, 8 * m + e) & 15u) | ((code(tau, 8 * m + 4 + e) & 15u) << 4)) << (8 * e);
                } else {
                    const int tau = i >> 1, h = i & 1;
                    for (int e = 0; e < 4; ++e) v |= ((code(tau, 4 * (4 * h + m) + e) ^ 0x80u) & 0xFFu) << (8 * e);
                }
                wd[m] = v;
            }
            *reinterpret_cast<uint4*>(out + size_t(sb) * out_sb + size_t(i) * 1024 + 16 * L) =
                make_uint4(wd[0], wd[1], wd[2], wd[3]);
        }
        for (int w = threadIdx.x; w < NSB * 64; w += blockDim.x) {
            const int sb = w >> 6, q = (w >> 4) & 3, tau = (w >> 2) & 3, v = w & 3;
            uint8_t* meta = out + size_t(sb) * out_sb + size_t(bits) * 1024;
            const int d = 4 * q + v, g = sb * 4 + tau;
            const uint16_t sv = sc[d * NT + g];
            meta[((q * 4 + tau) * 4 + v) * 2] = uint8_t(sv & 0xFF);
            meta[((q * 4 + tau) * 4 + v) * 2 + 1] = uint8_t(sv >> 8);
            meta[128 + (q * 4 + tau) * 4 + v] = zr[d * NT + g];
        }
        __syncthreads();
    }
}

}  // namespace

hipError_t launch_relayout(const uint8_t* src, uint8_t* dst, int R, int K, int bits, int gate_up, hipStream_t st) {
    const int nstrips = R / 16;
    const size_t lds = size_t(16) * K + size_t(16) * (K / GROUP) * 3;
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(relayout_kernel),
                                       hipFuncAttributeMaxDynamicSharedMemorySize, int(lds));
    if (e != hipSuccess) return e;
    const int grid = nstrips < 4096 ? nstrips : 4096;
    relayout_kernel<<<grid, 256, lds, st>>>(src, dst, nstrips, K, bits, gate_up);
    return hipGetLastError();
}

}  // namespace llmoe
