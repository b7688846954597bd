// INT4 group-32 weight formats: loader/repacker kernels and the bit-exact dequant.
//
// Row-packed layout used by every INT4 kernel in this library (per output row n,
// G = K/32 groups):
//   qw  uint32 [N, K/8]  group g = words 4g..4g+3; word j covers k = 32g + 8j + t and holds
//                        the code of t = 2i at bits [4i, 4i+4) and of t = 2i+1 at bits
//                        [16+4i, 20+4i), so one mask+or per pair of codes yields two bf16
//                        lanes for v_dot2_f32_bf16.
//   sc  bf16   [N, G]
//   zp  uint8  [N, G/2]  blocks of 128 groups: for block c (r = min(128, G - 128c) groups)
//                        byte 64c + b = z[128c + b] | z[128c + r/2 + b] << 4, so a GEMV lane
//                        owning groups l and l + 64 of a 128-group slice reads one byte.
// w[n, k] = bf16_rne(float(q - z) * float(s))  -- src/moss_tts/_runtime/calibrated_quant.py:41-42.
#include "common.h"

namespace moss {
namespace {

// GPTQ word (code of t at bits 4t) -> row-packed word.  The same permutation maps one
// little-endian u32 of the reference's signed export (byte i = codes 2i | 2i+1 << 4,
// src/moss_tts/calibration.py:190-191) onto the row-packed order.
__device__ __forceinline__ uint32_t to_rowpack(uint32_t w) {
    uint32_t even = w & 0x0f0f0f0fu;          // t = 0,2,4,6 at bits 0,8,16,24
    uint32_t odd = (w >> 4) & 0x0f0f0f0fu;    // t = 1,3,5,7 at bits 0,8,16,24
    // compact the four byte-spaced nibbles of each into 16 bits
    uint32_t e = (even | (even >> 4)) & 0x00ff00ffu;
    e = (e | (e >> 8)) & 0x0000ffffu;
    uint32_t o = (odd | (odd >> 4)) & 0x00ff00ffu;
    o = (o | (o >> 8)) & 0x0000ffffu;
    return e | (o << 16);
}

__device__ __forceinline__ uint32_t rowpack_code(uint32_t w, int t) {
    return (t & 1) ? (w >> (16 + 4 * (t >> 1))) & 15u : (w >> (4 * (t >> 1))) & 15u;
}

// (byte index, group of its low nibble, group of its high nibble) for zero byte i of a row
__device__ __forceinline__ void zero_byte_groups(int i, int G, int& lo, int& hi) {
    const int c0 = (i >> 6) << 7, r = min(128, G - c0), b = i - (c0 >> 1);
    lo = c0 + b;
    hi = c0 + (r >> 1) + b;
}

constexpr int kTile = 64;

// qweight int32 [K8, N] -> qw uint32 [N, K8]: LDS-tiled transpose + nibble permutation.
__global__ __launch_bounds__(256) void repack_gptq_qweight(const uint32_t* __restrict__ in,
                                                           uint32_t* __restrict__ out, int K8, int N) {
    __shared__ uint32_t tile[kTile][kTile + 1];
    const int n0 = blockIdx.x * kTile, w0 = blockIdx.y * kTile;
    const int tx = threadIdx.x & 63, ty = threadIdx.x >> 6;
    for (int r = ty; r < kTile; r += 4) {
        const int w = w0 + r, n = n0 + tx;
        if (w < K8 && n < N) tile[r][tx] = in[(size_t)w * N + n];
    }
    __syncthreads();
    for (int r = ty; r < kTile; r += 4) {
        const int n = n0 + r, w = w0 + tx;
        if (n < N && w < K8) out[(size_t)n * K8 + w] = to_rowpack(tile[tx][r]);
    }
}

// scales bf16 [G, N] -> [N, G]
__global__ __launch_bounds__(256) void transpose_u16(const uint16_t* __restrict__ in,
                                                     uint16_t* __restrict__ out, int R, int C) {
    __shared__ uint16_t tile[kTile][kTile + 1];
    const int c0 = blockIdx.x * kTile, r0 = blockIdx.y * kTile;
    const int tx = threadIdx.x & 63, ty = threadIdx.x >> 6;
    for (int r = ty; r < kTile; r += 4) {
        const int rr = r0 + r, cc = c0 + tx;
        if (rr < R && cc < C) tile[r][tx] = in[(size_t)rr * C + cc];
    }
    __syncthreads();
    for (int r = ty; r < kTile; r += 4) {
        const int cc = c0 + r, rr = r0 + tx;
        if (cc < C && rr < R) out[(size_t)cc * R + rr] = tile[tx][r];
    }
}

// qzeros int32 [G, N/8] -> zp uint8 [N, G/2]
__global__ __launch_bounds__(256) void repack_gptq_zeros(const uint32_t* __restrict__ qz,
                                                         uint8_t* __restrict__ zp, int G, int N) {
    const int h = G >> 1;
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (size_t)N * h) return;
    const int n = (int)(i / h), b = (int)(i % h);
    int glo, ghi;
    zero_byte_groups(b, G, glo, ghi);
    const int sh = 4 * (n & 7);
    const uint32_t lo = (qz[(size_t)glo * (N / 8) + n / 8] >> sh) & 15u;
    const uint32_t hi = (qz[(size_t)ghi * (N / 8) + n / 8] >> sh) & 15u;
    zp[i] = (uint8_t)(lo | (hi << 4));
}

// Reference signed export u8 [N, K/2] (viewed as u32 [N, K8]) -> qw with q = u ^ 8, z = 8.
__global__ __launch_bounds__(256) void import_signed_words(const uint32_t* __restrict__ in,
                                                           uint32_t* __restrict__ out, size_t words) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < words) out[i] = to_rowpack(in[i]) ^ 0x88888888u;
}

__global__ __launch_bounds__(256) void fill_u8(uint8_t* __restrict__ p, uint8_t v, size_t n) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) p[i] = v;
}

// qw [N, K8] -> codes u8 [N, K]
__global__ __launch_bounds__(256) void unpack_codes(const uint32_t* __restrict__ qw,
                                                    uint8_t* __restrict__ codes, size_t words) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= words) return;
    const uint32_t w = qw[i];
    uint32_t lo = 0, hi = 0;
#pragma unroll
    for (int t = 0; t < 4; ++t) lo |= rowpack_code(w, t) << (8 * t);
#pragma unroll
    for (int t = 0; t < 4; ++t) hi |= rowpack_code(w, t + 4) << (8 * t);
    reinterpret_cast<uint2*>(codes)[i] = make_uint2(lo, hi);
}

// (qw, sc, zp) -> bf16 [N, K]; one thread per packed word (8 weights, one 16-byte store).
__global__ __launch_bounds__(256) void dequant_bf16(const uint32_t* __restrict__ qw,
                                                    const uint16_t* __restrict__ sc,
                                                    const uint8_t* __restrict__ zp,
                                                    uint16_t* __restrict__ out, int K, int N) {
    const int K8 = K >> 3, G = K >> 5;
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (size_t)N * K8) return;
    const int n = (int)(i / K8), w = (int)(i % K8), g = w >> 2;
    const uint32_t word = qw[i];
    const float s = bf16_bits(sc[(size_t)n * G + g]);
    const int z = (int)zero_of_group(zp + (size_t)n * (G >> 1), g, G);
    uint32_t o[4];
#pragma unroll
    for (int p = 0; p < 4; ++p) {
        const float a = (float)((int)rowpack_code(word, 2 * p) - z) * s;
        const float b = (float)((int)rowpack_code(word, 2 * p + 1) - z) * s;
        o[p] = pack_bf16x2(a, b);
    }
    reinterpret_cast<uint4*>(out)[i] = make_uint4(o[0], o[1], o[2], o[3]);
}

// Min-max RTN quantizer (fp32 weights [N, K]) straight into the row-packed layout.
// One thread per zero byte (its two groups), so no two threads share a byte.
__device__ __forceinline__ void quantize_group(const float* __restrict__ wg, uint32_t* __restrict__ qwg,
                                               uint16_t* __restrict__ s_out, uint32_t* z_out) {
    float v[32];
#pragma unroll
    for (int c = 0; c < 8; ++c) {
        const float4 t = reinterpret_cast<const float4*>(wg)[c];
        v[4 * c] = t.x; v[4 * c + 1] = t.y; v[4 * c + 2] = t.z; v[4 * c + 3] = t.w;
    }
    float lo = v[0], hi = v[0];
#pragma unroll
    for (int t = 1; t < 32; ++t) { lo = fminf(lo, v[t]); hi = fmaxf(hi, v[t]); }
    const float s32 = fmaxf((hi - lo) / 15.0f, 1e-8f);
    const uint16_t sb = f32_to_bf16(s32);
    const float s = bf16_bits(sb);
    const float z = fminf(fmaxf(rintf(-lo / s), 0.0f), 15.0f);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        uint32_t word = 0;
#pragma unroll
        for (int t = 0; t < 8; ++t) {
            const float q = fminf(fmaxf(rintf(v[8 * j + t] / s) + z, 0.0f), 15.0f);
            const int sh = (t & 1) ? 16 + 4 * (t >> 1) : 4 * (t >> 1);
            word |= ((uint32_t)q) << sh;
        }
        qwg[j] = word;
    }
    *s_out = sb;
    *z_out = (uint32_t)z;
}

// Symmetric RTN against static scales (src/moss_tts/_runtime/calibrated_quant.py:36-38 and the
// no-Hessian rounding of :74-77): s = bf16(max(max|w|, 1e-8) / 7), c = clamp(rint(w / s), -7, 7)
// (IEEE division, ties to even), stored as q = c + 8 with z = 8, so (q - z) s = c s.
__device__ __forceinline__ void quantize_group_symmetric(const float* __restrict__ wg, uint32_t* __restrict__ qwg,
                                                         uint16_t* __restrict__ s_out) {
    float v[32];
#pragma unroll
    for (int c = 0; c < 8; ++c) {
        const float4 t = reinterpret_cast<const float4*>(wg)[c];
        v[4 * c] = t.x; v[4 * c + 1] = t.y; v[4 * c + 2] = t.z; v[4 * c + 3] = t.w;
    }
    float amax = 0.f;
#pragma unroll
    for (int t = 0; t < 32; ++t) amax = fmaxf(amax, fabsf(v[t]));
    const uint16_t sb = f32_to_bf16(fmaxf(amax, 1e-8f) / 7.0f);
    const float s = bf16_bits(sb);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        uint32_t word = 0;
#pragma unroll
        for (int t = 0; t < 8; ++t) {
            const float c = fminf(fmaxf(rintf(v[8 * j + t] / s), -7.0f), 7.0f);
            const int sh = (t & 1) ? 16 + 4 * (t >> 1) : 4 * (t >> 1);
            word |= ((uint32_t)((int)c + 8)) << sh;
        }
        qwg[j] = word;
    }
    *s_out = sb;
}

__global__ __launch_bounds__(256) void quantize_symmetric(const float* __restrict__ w, uint32_t* __restrict__ qw,
                                                          uint16_t* __restrict__ sc, uint8_t* __restrict__ zp, int K,
                                                          int N) {
    const int G = K >> 5, h = G >> 1;
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (size_t)N * h) return;
    const int n = (int)(i / h), b = (int)(i % h);
    int glo, ghi;
    zero_byte_groups(b, G, glo, ghi);
    quantize_group_symmetric(w + (size_t)n * K + 32 * glo, qw + (size_t)n * (K >> 3) + 4 * glo, sc + (size_t)n * G + glo);
    quantize_group_symmetric(w + (size_t)n * K + 32 * ghi, qw + (size_t)n * (K >> 3) + 4 * ghi, sc + (size_t)n * G + ghi);
    zp[i] = 0x88;
}

__global__ __launch_bounds__(256) void quantize_minmax(const float* __restrict__ w, uint32_t* __restrict__ qw,
                                                       uint16_t* __restrict__ sc, uint8_t* __restrict__ zp,
                                                       int K, int N) {
    const int G = K >> 5, h = G >> 1;
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (size_t)N * h) return;
    const int n = (int)(i / h), b = (int)(i % h);
    int glo, ghi;
    zero_byte_groups(b, G, glo, ghi);
    uint32_t z0, z1;
    quantize_group(w + (size_t)n * K + 32 * glo, qw + (size_t)n * (K >> 3) + 4 * glo, sc + (size_t)n * G + glo, &z0);
    quantize_group(w + (size_t)n * K + 32 * ghi, qw + (size_t)n * (K >> 3) + 4 * ghi, sc + (size_t)n * G + ghi, &z1);
    zp[i] = (uint8_t)(z0 | (z1 << 4));
}

inline unsigned blocks_for(size_t n, int threads) { return (unsigned)((n + threads - 1) / threads); }

}  // namespace
}  // namespace moss

using namespace moss;

MOSS_API int moss_w4g32_repack_gptq(const void* qweight, const void* scales, const void* qzeros, void* qw,
                                    void* sc, void* zp, int K, int N, void* stream) {
    MOSS_CHECK_ARG(qweight && scales && qzeros && qw && sc && zp);
    MOSS_CHECK_ARG(K > 0 && N > 0 && K % 64 == 0 && N % 8 == 0);
    const int K8 = K / 8, G = K / 32;
    hipStream_t st = (hipStream_t)stream;
    dim3 grid_q((N + kTile - 1) / kTile, (K8 + kTile - 1) / kTile);
    hipLaunchKernelGGL(repack_gptq_qweight, grid_q, dim3(256), 0, st, (const uint32_t*)qweight, (uint32_t*)qw, K8, N);
    dim3 grid_s((N + kTile - 1) / kTile, (G + kTile - 1) / kTile);
    hipLaunchKernelGGL(transpose_u16, grid_s, dim3(256), 0, st, (const uint16_t*)scales, (uint16_t*)sc, G, N);
    const size_t nz = (size_t)N * (G / 2);
    hipLaunchKernelGGL(repack_gptq_zeros, dim3(blocks_for(nz, 256)), dim3(256), 0, st, (const uint32_t*)qzeros,
                       (uint8_t*)zp, G, N);
    return moss_launch_status();
}

MOSS_API int moss_w4g32_import_signed(const void* packed, void* qw, void* zp, int K, int N, void* stream) {
    MOSS_CHECK_ARG(packed && qw && zp && K > 0 && N > 0 && K % 64 == 0);
    MOSS_CHECK_ARG(MOSS_ALIGNED(packed, 4) && MOSS_ALIGNED(qw, 4));
    hipStream_t st = (hipStream_t)stream;
    const size_t words = (size_t)N * (K / 8);
    hipLaunchKernelGGL(import_signed_words, dim3(blocks_for(words, 256)), dim3(256), 0, st,
                       (const uint32_t*)packed, (uint32_t*)qw, words);
    const size_t nz = (size_t)N * (K / 64);
    hipLaunchKernelGGL(fill_u8, dim3(blocks_for(nz, 256)), dim3(256), 0, st, (uint8_t*)zp, (uint8_t)0x88, nz);
    return moss_launch_status();
}

MOSS_API int moss_w4g32_unpack_codes(const void* qw, void* codes, int K, int N, void* stream) {
    MOSS_CHECK_ARG(qw && codes && K > 0 && N > 0 && K % 64 == 0 && MOSS_ALIGNED(codes, 8));
    const size_t words = (size_t)N * (K / 8);
    hipLaunchKernelGGL(unpack_codes, dim3(blocks_for(words, 256)), dim3(256), 0, (hipStream_t)stream,
                       (const uint32_t*)qw, (uint8_t*)codes, words);
    return moss_launch_status();
}

MOSS_API int moss_w4g32_dequant_bf16(const void* qw, const void* sc, const void* zp, void* w, int K, int N,
                                     void* stream) {
    MOSS_CHECK_ARG(qw && sc && zp && w && K > 0 && N > 0 && K % 64 == 0 && MOSS_ALIGNED(w, 16));
    const size_t words = (size_t)N * (K / 8);
    hipLaunchKernelGGL(dequant_bf16, dim3(blocks_for(words, 256)), dim3(256), 0, (hipStream_t)stream,
                       (const uint32_t*)qw, (const uint16_t*)sc, (const uint8_t*)zp, (uint16_t*)w, K, N);
    return moss_launch_status();
}

MOSS_API int moss_w4g32_quantize_minmax(const void* w, void* qw, void* sc, void* zp, int K, int N, void* stream) {
    MOSS_CHECK_ARG(w && qw && sc && zp && K > 0 && N > 0 && K % 64 == 0 && MOSS_ALIGNED(w, 16));
    const size_t threads = (size_t)N * (K / 64);
    hipLaunchKernelGGL(quantize_minmax, dim3(blocks_for(threads, 256)), dim3(256), 0, (hipStream_t)stream,
                       (const float*)w, (uint32_t*)qw, (uint16_t*)sc, (uint8_t*)zp, K, N);
    return moss_launch_status();
}

MOSS_API int moss_w4g32_quantize_symmetric(const void* w, void* qw, void* sc, void* zp, int K, int N, void* stream) {
    MOSS_CHECK_ARG(w && qw && sc && zp && K > 0 && N > 0 && K % 64 == 0 && MOSS_ALIGNED(w, 16));
    const size_t threads = (size_t)N * (K / 64);
    hipLaunchKernelGGL(quantize_symmetric, dim3(blocks_for(threads, 256)), dim3(256), 0, (hipStream_t)stream,
                       (const float*)w, (uint32_t*)qw, (uint16_t*)sc, (uint8_t*)zp, K, N);
    return moss_launch_status();
}
