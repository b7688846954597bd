// FP8 E4M3 (OCP) weight-only linear: y[m, n] = bf16(s[n] * sum_k f32(w[n, k]) * x[m, k]),
// w e4m3 [N, K] row-major bytes, s fp32 [N] (or 1 when absent), x and y bf16, fp32 accumulate;
// and the fused gate||up form that rounds gate and up to bf16, then bf16(silu(gate)) * up.
//
// Reference: src/moss_tts/_runtime/fused_mlp.py:7-23 (`_fp8_silu_gemv`: per-row sums of
// f32(w) * f32(x), times the optional row scale, rounded to bf16; SiLU rounded to bf16; the
// product stored as bf16) and its launcher fused_mlp.py:26-30.
//
// Every e4m3 value is exactly representable in bf16 (4-bit significand, exponents 2^-9..2^8),
// so weights are converted with v_cvt_scalef32_pk_bf16_fp8 (scale 1) and meet x in
// v_dot2_f32_bf16: no rounding happens before the fp32 accumulation, as in the reference.
//
// Decode (M = 1): one wave owns R rows; lane l reads bytes 16 l + 1024 j of each row
// (one global_load_dwordx4 per 1 KiB slab of the row), so every wave load is 1 KiB
// contiguous.  The lane's 16 x values per slab stay in VGPRs for all R rows.  Prefill (M > 1)
// goes to the MFMA GEMM (w4g32_gemm.hip) with the e4m3 -> bf16 conversion in its B-tile
// producer and the row scale in its epilogue.
#include "common.h"

namespace moss {

int fp8_gemm_launch(const void* x, const void* w, const float* row_scale, void* y, int M, int K, int N, void* ws,
                    long long ws_bytes, hipStream_t stream);

namespace {

typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));

template <bool HI>
__device__ __forceinline__ uint32_t fp8x2_bf16x2(uint32_t w) {
    return __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w, 1.0f, HI));
}

// One 16-byte slab: 16 weights against 8 packed x pairs.
__device__ __forceinline__ float slab_dot(const uint4& w, const uint32_t* xv, float acc) {
    const uint32_t words[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
    for (int c = 0; c < 4; ++c) {
        acc = dot2_bf16(fp8x2_bf16x2<false>(words[c]), xv[2 * c], acc);
        acc = dot2_bf16(fp8x2_bf16x2<true>(words[c]), xv[2 * c + 1], acc);
    }
    return acc;
}

// KC = ceil(K / 1024) slabs per lane; FULL: K == 1024 KC (no per-lane bound checks).
template <int KC, int R, bool PAIRED, bool FULL>
__global__ __launch_bounds__(256) void fp8_gemv_kernel(const uint16_t* __restrict__ x, const uint8_t* __restrict__ w,
                                                       const float* __restrict__ scale, uint16_t* __restrict__ y,
                                                       int K, int n_out) {
    const int lane = threadIdx.x & (kWave - 1);
    const int wave = __builtin_amdgcn_readfirstlane(blockIdx.x * (blockDim.x / kWave) + (threadIdx.x / kWave));
    const int row0 = wave * R;
    if (row0 >= n_out) return;  // wave-uniform

    constexpr int NR = PAIRED ? 2 * R : R;
    uint4 rows[NR][KC];
#pragma unroll
    for (int r = 0; r < NR; ++r) {
        const int local = PAIRED ? (r % R) : r;
        const int n = min(row0 + local, n_out - 1) + ((PAIRED && r >= R) ? n_out : 0);
        const uint8_t* row = w + (size_t)n * K;
#pragma unroll
        for (int j = 0; j < KC; ++j) {
            const int k = 1024 * j + 16 * lane;
            if (FULL || k < K) {
                const u32x4_t v = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(row + k));
                rows[r][j] = make_uint4(v.x, v.y, v.z, v.w);
            } else {
                rows[r][j] = make_uint4(0u, 0u, 0u, 0u);
            }
        }
    }
    uint32_t xv[KC][8];
#pragma unroll
    for (int j = 0; j < KC; ++j) {
        const int k = 1024 * j + 16 * lane;
        if (FULL || k < K) {
            const uint4* p = reinterpret_cast<const uint4*>(x + k);
            const uint4 a = p[0], b = p[1];
            xv[j][0] = a.x; xv[j][1] = a.y; xv[j][2] = a.z; xv[j][3] = a.w;
            xv[j][4] = b.x; xv[j][5] = b.y; xv[j][6] = b.z; xv[j][7] = b.w;
        } else {
#pragma unroll
            for (int c = 0; c < 8; ++c) xv[j][c] = 0u;
        }
    }
    float out[NR];
#pragma unroll
    for (int r = 0; r < NR; ++r) {
        float acc = 0.f;
#pragma unroll
        for (int j = 0; j < KC; ++j) acc = slab_dot(rows[r][j], xv[j], acc);
        out[r] = wave_sum(acc);
    }
    if (lane == 0) {
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const int n = row0 + r;
            if (n >= n_out) continue;
            const float a = out[r] * (scale ? scale[n] : 1.0f);
            if constexpr (PAIRED) {
                const float b = out[R + r] * (scale ? scale[n + n_out] : 1.0f);
                y[n] = silu_mul_rounded_bits(a, b);
            } else {
                y[n] = f32_to_bf16(a);
            }
        }
    }
}

template <bool PAIRED>
int launch_gemv(const void* x, const void* w, const float* scale, void* y, int K, int n_out, int rows,
                hipStream_t st) {
    const int KC = (K + 1023) / 1024;
    const bool full = K == 1024 * KC;
    if (rows <= 0) rows = KC <= 4 ? 2 : 1;
    const auto* xp = (const uint16_t*)x;
    const auto* wp = (const uint8_t*)w;
    auto* yp = (uint16_t*)y;
    const int waves = (n_out + rows - 1) / rows;
    const dim3 grid((waves + 3) / 4), block(256);
#define MOSS_F8(KCV, RV)                                                                                     \
    if (KC == KCV && rows == RV) {                                                                           \
        if (full)                                                                                            \
            hipLaunchKernelGGL((fp8_gemv_kernel<KCV, RV, PAIRED, true>), grid, block, 0, st, xp, wp, scale, yp, \
                               K, n_out);                                                                    \
        else                                                                                                 \
            hipLaunchKernelGGL((fp8_gemv_kernel<KCV, RV, PAIRED, false>), grid, block, 0, st, xp, wp, scale,  \
                               yp, K, n_out);                                                                \
        return moss_launch_status();                                                                         \
    }
#define MOSS_F8_R(KCV) MOSS_F8(KCV, 1) MOSS_F8(KCV, 2) MOSS_F8(KCV, 4)
    MOSS_F8_R(1) MOSS_F8_R(2) MOSS_F8_R(3) MOSS_F8_R(4)
    MOSS_F8(5, 1) MOSS_F8(6, 1) MOSS_F8(7, 1) MOSS_F8(8, 1) MOSS_F8(5, 2) MOSS_F8(6, 2) MOSS_F8(7, 2) MOSS_F8(8, 2)
    MOSS_F8(9, 1) MOSS_F8(10, 1) MOSS_F8(11, 1) MOSS_F8(12, 1)
    MOSS_F8(13, 1) MOSS_F8(14, 1) MOSS_F8(15, 1) MOSS_F8(16, 1)
#undef MOSS_F8_R
#undef MOSS_F8
    return (int)hipErrorInvalidValue;
}

__global__ __launch_bounds__(256) void fp8_to_bf16_kernel(const uint32_t* __restrict__ w, uint2* __restrict__ out,
                                                          size_t words) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < words) out[i] = make_uint2(fp8x2_bf16x2<false>(w[i]), fp8x2_bf16x2<true>(w[i]));
}

}  // namespace
}  // namespace moss

using namespace moss;

MOSS_API int moss_fp8_linear(const void* x, const void* w, const void* scale, void* y, int M, int K, int N,
                             int rows_per_wave, void* workspace, long long workspace_bytes, void* stream) {
    MOSS_CHECK_ARG(x && w && y && M > 0 && N > 0 && K > 0);
    MOSS_CHECK_ARG(MOSS_ALIGNED(x, 16) && MOSS_ALIGNED(w, 16) && MOSS_ALIGNED(y, 2));
    if (M == 1) {
        MOSS_CHECK_ARG(K % 16 == 0 && K <= 16384);
        return launch_gemv<false>(x, w, (const float*)scale, y, K, N, rows_per_wave, (hipStream_t)stream);
    }
    MOSS_CHECK_ARG(K % 64 == 0 && workspace_bytes >= 0);
    return fp8_gemm_launch(x, w, (const float*)scale, y, M, K, N, workspace, workspace_bytes, (hipStream_t)stream);
}

MOSS_API int moss_fp8_gateup_silu(const void* x, const void* w, const void* scale, void* y, int M, int K,
                                  int N_half, int rows_per_wave, void* stream) {
    MOSS_CHECK_ARG(x && w && y && M == 1 && N_half > 0 && K > 0 && K % 16 == 0 && K <= 16384);
    MOSS_CHECK_ARG(MOSS_ALIGNED(x, 16) && MOSS_ALIGNED(w, 16) && MOSS_ALIGNED(y, 2));
    return launch_gemv<true>(x, w, (const float*)scale, y, K, N_half, rows_per_wave, (hipStream_t)stream);
}

MOSS_API int moss_fp8_to_bf16(const void* w, void* out, long long count, void* stream) {
    MOSS_CHECK_ARG(w && out && count > 0 && count % 4 == 0);
    MOSS_CHECK_ARG(MOSS_ALIGNED(w, 4) && MOSS_ALIGNED(out, 8));
    const size_t words = (size_t)count / 4;
    hipLaunchKernelGGL(fp8_to_bf16_kernel, dim3((unsigned)((words + 255) / 256)), dim3(256), 0, (hipStream_t)stream,
                       (const uint32_t*)w, (uint2*)out, words);
    return moss_launch_status();
}
