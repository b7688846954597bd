// Batch-1 GEMV with bf16 weights, optionally behind the fused (add+)RMSNorm: the output heads.
//
// y[n] = bf16(sum_k f32(w[n,k]) * f32(x[k]))     (fp32 accumulate, one rounding at the end)
//
// The reference keeps the 32 audio-codebook heads and the two text-head rows in bf16 and applies
// them with F.linear / its Triton GEMV (src/moss_tts/_runtime/llm.py:188-191,270-279;
// src/moss_tts/_runtime/kernels.py:93-108).  At 268 MB per decode step this is the largest single
// weight read after the layers, so the kernel is a plain HBM stream: one wave owns R rows, lane l
// reads the 16-byte chunks l + 64 c of each row (every global_load_dwordx4 of a wave is 1 KiB
// contiguous, non-temporal: each weight byte is read once), keeps the matching x chunks in VGPRs
// for all R rows, and multiplies pairs with v_dot2_f32_bf16 (bf16 x bf16 products are exact in
// fp32).  Rows are reduced with the fixed-order DPP sum, so results are deterministic.
#include "common.h"
#include "norm_fused.h"

namespace moss {
namespace {

typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));

// KC = K / 512 chunks of 8 values per lane.  NORM as in norm_fused.h (0: x used as is).
template <int KC, int R, int NORM>
__global__ __launch_bounds__(256) void bf16_gemv_kernel(const uint16_t* __restrict__ x, const uint4* __restrict__ w,
                                                        uint16_t* __restrict__ y, int N, NormArgs na) {
    constexpr int K8 = KC * kWave;  // 16-byte chunks per row
    const int lane = threadIdx.x & (kWave - 1);
    const int wave = __builtin_amdgcn_readfirstlane(blockIdx.x * 4 + (threadIdx.x / kWave));
    const int row0 = wave * R;
    if (NORM == 0 && row0 >= N) return;  // wave-uniform

    NormLoad<(NORM > 0 ? KC / 4 : 1)> nl;
    uint4 xv[KC];
    if constexpr (NORM > 0) {
        norm_load<NORM, KC / 4>(nl, x, na);
    } else {
#pragma unroll
        for (int c = 0; c < KC; ++c) xv[c] = reinterpret_cast<const uint4*>(x)[lane + kWave * c];
    }
    uint4 wr[R][KC];
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const size_t n = (size_t)min(row0 + r, N - 1);
#pragma unroll
        for (int c = 0; c < KC; ++c) {
            const u32x4_t v = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(w + n * K8 + lane + kWave * c));
            wr[r][c] = make_uint4(v.x, v.y, v.z, v.w);
        }
    }
    if constexpr (NORM > 0) {
        __shared__ __attribute__((aligned(16))) uint16_t xn[512 * KC];
        __shared__ float red[4];
        norm_into_lds<NORM, KC / 4>(nl, na, xn, red, 512 * KC);
        if (row0 >= N) return;  // after the workgroup's barriers
#pragma unroll
        for (int c = 0; c < KC; ++c) xv[c] = reinterpret_cast<const uint4*>(xn)[lane + kWave * c];
    }
    float out[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
        float acc = 0.f;
#pragma unroll
        for (int c = 0; c < KC; ++c) {
            acc = dot2_bf16(wr[r][c].x, xv[c].x, acc);
            acc = dot2_bf16(wr[r][c].y, xv[c].y, acc);
            acc = dot2_bf16(wr[r][c].z, xv[c].z, acc);
            acc = dot2_bf16(wr[r][c].w, xv[c].w, acc);
        }
        out[r] = wave_sum(acc);
    }
    if (lane == 0) {
#pragma unroll
        for (int r = 0; r < R; ++r)
            if (row0 + r < N) y[row0 + r] = f32_to_bf16(out[r]);
    }
}

template <int KC, int NORM>
int launch_kc(const void* x, const void* w, void* y, int N, int rows, const NormArgs& na, hipStream_t st) {
    const int waves = (N + rows - 1) / rows;
    const dim3 grid((waves + 3) / 4), block(256);
    const auto* xp = (const uint16_t*)x;
    const auto* wp = (const uint4*)w;
    auto* yp = (uint16_t*)y;
    switch (rows) {
        case 1: hipLaunchKernelGGL((bf16_gemv_kernel<KC, 1, NORM>), grid, block, 0, st, xp, wp, yp, N, na); break;
        case 2: hipLaunchKernelGGL((bf16_gemv_kernel<KC, 2, NORM>), grid, block, 0, st, xp, wp, yp, N, na); break;
        case 4: hipLaunchKernelGGL((bf16_gemv_kernel<KC, 4, NORM>), grid, block, 0, st, xp, wp, yp, N, na); break;
        default: return (int)hipErrorInvalidValue;
    }
    return moss_launch_status();
}

template <int NORM>
int launch_bf16_gemv(const void* x, const void* w, void* y, int K, int N, int rows, const NormArgs& na,
                     hipStream_t st) {
    if (rows == 0) rows = 2;
    switch (K / 512) {
        case 4: return launch_kc<4, NORM>(x, w, y, N, rows, na, st);
        case 8: return launch_kc<8, NORM>(x, w, y, N, rows, na, st);
        case 12: return launch_kc<12, NORM>(x, w, y, N, rows, na, st);
        case 16: return launch_kc<16, NORM>(x, w, y, N, rows, na, st);
        default: break;
    }
    if constexpr (NORM == 0) {
        switch (K / 512) {
            case 1: return launch_kc<1, 0>(x, w, y, N, rows, na, st);
            case 2: return launch_kc<2, 0>(x, w, y, N, rows, na, st);
            case 3: return launch_kc<3, 0>(x, w, y, N, rows, na, st);
            case 5: return launch_kc<5, 0>(x, w, y, N, rows, na, st);
            case 6: return launch_kc<6, 0>(x, w, y, N, rows, na, st);
            case 7: return launch_kc<7, 0>(x, w, y, N, rows, na, st);
            default: break;
        }
    }
    return (int)hipErrorInvalidValue;
}

}  // namespace
}  // namespace moss

using namespace moss;

MOSS_API int moss_bf16_gemv(const void* x, const void* w, void* y, int K, int N, int rows_per_wave, void* stream) {
    MOSS_CHECK_ARG(x && w && y && N > 0 && K > 0 && K % 512 == 0 && K <= 8192 && K / 512 != 9 && K / 512 != 10 &&
                   K / 512 != 11 && K / 512 != 13 && K / 512 != 14 && K / 512 != 15);
    MOSS_CHECK_ARG(rows_per_wave == 0 || rows_per_wave == 1 || rows_per_wave == 2 || rows_per_wave == 4);
    MOSS_CHECK_ARG(MOSS_ALIGNED(x, 16) && MOSS_ALIGNED(w, 16));
    return launch_bf16_gemv<0>(x, w, y, K, N, rows_per_wave, NormArgs{}, (hipStream_t)stream);
}

MOSS_API int moss_bf16_norm_gemv(const void* x, const void* res, const void* norm_w, void* sum_out, float eps,
                                 const void* w, void* y, int K, int N, int rows_per_wave, void* stream) {
    if (int rc = moss_check_norm_args(x, res, norm_w, sum_out, K, eps)) return rc;
    MOSS_CHECK_ARG(w && y && N > 0 && MOSS_ALIGNED(w, 16));
    MOSS_CHECK_ARG(rows_per_wave == 0 || rows_per_wave == 1 || rows_per_wave == 2 || rows_per_wave == 4);
    const NormArgs na{(const uint16_t*)res, (const uint16_t*)norm_w, (uint16_t*)sum_out, eps};
    if (res) return launch_bf16_gemv<2>(x, w, y, K, N, rows_per_wave, na, (hipStream_t)stream);
    return launch_bf16_gemv<1>(x, w, y, K, N, rows_per_wave, na, (hipStream_t)stream);
}
