// Prefill GEMM on MFMA: Y[M, N] = X[M, K] . W[N, K]^T, bf16 in/out, fp32 accumulate, for
// INT4 group-32 weights (row-packed) and for FP8 E4M3 weights with fp32 row scales.
//
// INT4: the reference keeps bf16 weights for prefill (src/moss_tts/_runtime/llm.py:29,84,130);
// its dequant-then-matmul (src/moss_tts/calibration.py:185-188) is the contract here.  Every
// weight is dequantized bit-exactly, bf16_rne((q - z) * s) as in
// src/moss_tts/_runtime/calibrated_quant.py:41-42, into LDS and then multiplied on the
// matrix cores (v_mfma_f32_32x32x16_bf16).
// FP8: every e4m3 value is a bf16 value, so the B-tile producer converts exactly
// (v_cvt_scalef32_pk_bf16_fp8, scale 1) and the row scale multiplies the fp32 sum in the
// epilogue (src/moss_tts/_runtime/fused_mlp.py:20-21).  The fp8 MFMA forms are not used:
// they would round the bf16 activations to e4m3 as well.
//
// Tile: BM x BN outputs per 256-thread workgroup (2 x 2 waves, each 2 x 2 MFMA tiles of
// 32 x 32), K in steps of 64 (two quantization groups).  Per step each thread dequantizes
// one 32-code group (or converts 32 e4m3 bytes) of one weight row and copies 32
// activations; the next step's global loads are issued into registers before the current
// step's MFMAs.
#include "common.h"

namespace moss {
namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));

constexpr int kBK = 64;
constexpr int kPad = 8;  // bf16 padding per LDS row: breaks the 128-byte bank period
constexpr int kLds = kBK + kPad;

enum WeightFormat { kInt4G32 = 0, kFp8E4M3 = 1 };

struct StepRegs {
    uint4 x[4];     // 32 activations of one X row
    uint4 w[2];     // INT4: w[0] = 32 codes of one weight row; FP8: 32 e4m3 bytes
    uint32_t s, z;  // INT4: its group's scale bits and zero point
};

template <int BM, int BN, int FMT>
__device__ __forceinline__ void load_step(StepRegs& r, const uint16_t* __restrict__ X, const uint4* __restrict__ qw,
                                          const uint16_t* __restrict__ sc, const uint8_t* __restrict__ zp, int M,
                                          int N, int K, int G, int m0, int n0, int k0, int tid) {
    const int row = tid >> 1, half = tid & 1;
    // activations: thread -> (row, 32-wide half of the step); rows beyond M read as zero
#pragma unroll
    for (int rr = 0; rr < BM / 128; ++rr) {
        const int m = m0 + row + 128 * rr;
        if (rr == 0) {
            if (m < M) {
                const uint4* p = reinterpret_cast<const uint4*>(X + (size_t)m * K + k0 + 32 * half);
#pragma unroll
                for (int c = 0; c < 4; ++c) r.x[c] = p[c];
            } else {
#pragma unroll
                for (int c = 0; c < 4; ++c) r.x[c] = make_uint4(0u, 0u, 0u, 0u);
            }
        }
    }
    // weights: thread -> (row, 32-wide half of the step)
    const int n = n0 + row;
    if constexpr (FMT == kInt4G32) {
        const int g = (k0 >> 5) + half;
        if (row < BN && n < N) {
            r.w[0] = qw[(size_t)n * G + g];
            r.s = sc[(size_t)n * G + g];
            r.z = zero_of_group(zp + (size_t)n * (G >> 1), g, G);
        } else {
            r.w[0] = make_uint4(0u, 0u, 0u, 0u);
            r.s = 0u;
            r.z = 0u;
        }
    } else {
        if (row < BN && n < N) {
            const uint4* p = reinterpret_cast<const uint4*>(reinterpret_cast<const uint8_t*>(qw) + (size_t)n * K + k0 +
                                                            32 * half);
            r.w[0] = p[0];
            r.w[1] = p[1];
        } else {
            r.w[0] = r.w[1] = make_uint4(0u, 0u, 0u, 0u);
        }
    }
}

// Two e4m3 codes (bytes 2p, 2p+1 of a word pair) -> bf16 pair; exact: every e4m3 value is a bf16 value.
template <bool HI>
__device__ __forceinline__ uint32_t fp8x2_to_bf16x2(uint32_t w) {
    return __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w, 1.0f, HI));
}

template <int BM, int BN, int FMT>
__device__ __forceinline__ void store_step(const StepRegs& r, uint16_t (*As)[kLds], uint16_t (*Bs)[kLds], int tid) {
    const int row = tid >> 1, half = tid & 1;
    uint4* a = reinterpret_cast<uint4*>(&As[row][32 * half]);
#pragma unroll
    for (int c = 0; c < 4; ++c) a[c] = r.x[c];
    if constexpr (FMT == kFp8E4M3) {
        if (row < BN) {
            const uint32_t words[8] = {r.w[0].x, r.w[0].y, r.w[0].z, r.w[0].w, r.w[1].x, r.w[1].y, r.w[1].z, r.w[1].w};
            uint32_t out[16];
#pragma unroll
            for (int c = 0; c < 8; ++c) {
                out[2 * c] = fp8x2_to_bf16x2<false>(words[c]);
                out[2 * c + 1] = fp8x2_to_bf16x2<true>(words[c]);
            }
            uint4* b = reinterpret_cast<uint4*>(&Bs[row][32 * half]);
#pragma unroll
            for (int c = 0; c < 4; ++c) b[c] = make_uint4(out[4 * c], out[4 * c + 1], out[4 * c + 2], out[4 * c + 3]);
        }
        return;
    } else if (row < BN) {
        uint32_t mask = 0x000F000Fu, bias_bits = 0x43004300u;
        asm volatile("" : "+v"(mask), "+v"(bias_bits));
        const uint32_t s_lo = r.s & 0xffffu, s_hi = s_lo << 16;
        const float bias = -(128.0f + (float)r.z) * bf16_bits((uint16_t)s_lo);
        const uint32_t words[4] = {r.w[0].x, r.w[0].y, r.w[0].z, r.w[0].w};
        uint32_t out[16];
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int i = 0; i < 4; ++i)
                out[4 * j + i] = dequant_pair_exact(((words[j] >> (4 * i)) & mask) | bias_bits, s_lo, s_hi, bias);
        uint4* b = reinterpret_cast<uint4*>(&Bs[row][32 * half]);
#pragma unroll
        for (int c = 0; c < 4; ++c) b[c] = make_uint4(out[4 * c], out[4 * c + 1], out[4 * c + 2], out[4 * c + 3]);
    }
}

// FMT == kFp8E4M3: qw is e4m3 [N, K] (row-major bytes), `row_scale` fp32 [N] or null.
template <int BM, int BN, int FMT>
__global__ __launch_bounds__(256) void w4g32_gemm_kernel(const uint16_t* __restrict__ X, const uint4* __restrict__ qw,
                                                         const uint16_t* __restrict__ sc,
                                                         const uint8_t* __restrict__ zp, uint16_t* __restrict__ Y,
                                                         int M, int N, int K, const float* __restrict__ row_scale) {
    static_assert(BM == 128 && (BN == 128 || BN == 64), "tile");
    constexpr int WN = BN / 2;             // wave tile columns (2 x 2 waves)
    constexpr int TN = WN / 32;            // 32-wide MFMA tiles per wave along N
    __shared__ __attribute__((aligned(16))) uint16_t As[BM][kLds];
    __shared__ __attribute__((aligned(16))) uint16_t Bs[BN][kLds];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    const int m0 = blockIdx.y * BM, n0 = blockIdx.x * BN;
    const int G = K >> 5, steps = K / kBK;

    f32x16_t acc[2][TN];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j)
#pragma unroll
            for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.f;

    StepRegs r;
    load_step<BM, BN, FMT>(r, X, qw, sc, zp, M, N, K, G, m0, n0, 0, tid);
    for (int st = 0; st < steps; ++st) {
        store_step<BM, BN, FMT>(r, As, Bs, tid);
        __syncthreads();
        if (st + 1 < steps) load_step<BM, BN, FMT>(r, X, qw, sc, zp, M, N, K, G, m0, n0, (st + 1) * kBK, tid);
#pragma unroll
        for (int kk = 0; kk < kBK / 16; ++kk) {
            const int kc = 16 * kk + 8 * (lane >> 5);
            bf16x8_t a[2], b[TN];
#pragma unroll
            for (int i = 0; i < 2; ++i)
                a[i] = *reinterpret_cast<const bf16x8_t*>(&As[64 * wm + 32 * i + (lane & 31)][kc]);
#pragma unroll
            for (int j = 0; j < TN; ++j)
                b[j] = *reinterpret_cast<const bf16x8_t*>(&Bs[WN * wn + 32 * j + (lane & 31)][kc]);
#pragma unroll
            for (int i = 0; i < 2; ++i)
#pragma unroll
                for (int j = 0; j < TN; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[i], b[j], acc[i][j], 0, 0, 0);
        }
        __syncthreads();
    }
    // C layout of a 32 x 32 tile: lane l, element e -> row 8 (e / 4) + 4 (l / 32) + e % 4, column l % 32
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) {
            const int n = n0 + WN * wn + 32 * j + (lane & 31);
            if (n >= N) continue;
            // FP8: the per-row scale multiplies the finished sum (src/moss_tts/_runtime/fused_mlp.py:20-21)
            const float rs = (FMT == kFp8E4M3 && row_scale) ? row_scale[n] : 1.0f;
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                const int m = m0 + 64 * wm + 32 * i + 8 * (e >> 2) + 4 * (lane >> 5) + (e & 3);
                if (m < M) Y[(size_t)m * N + n] = f32_to_bf16(FMT == kFp8E4M3 ? acc[i][j][e] * rs : acc[i][j][e]);
            }
        }
}

template <int FMT>
int launch_gemm(const void* x, const void* qw, const void* sc, const void* zp, void* y, int M, int K, int N,
                const float* row_scale, hipStream_t st) {
    const int mt = (M + 127) / 128;
    // wide tiles when they already give one workgroup per CU, narrow ones otherwise
    if ((long)mt * ((N + 127) / 128) >= 256) {
        hipLaunchKernelGGL((w4g32_gemm_kernel<128, 128, FMT>), dim3((N + 127) / 128, mt), dim3(256), 0, st,
                           (const uint16_t*)x, (const uint4*)qw, (const uint16_t*)sc, (const uint8_t*)zp,
                           (uint16_t*)y, M, N, K, row_scale);
    } else {
        hipLaunchKernelGGL((w4g32_gemm_kernel<128, 64, FMT>), dim3((N + 63) / 64, mt), dim3(256), 0, st,
                           (const uint16_t*)x, (const uint4*)qw, (const uint16_t*)sc, (const uint8_t*)zp,
                           (uint16_t*)y, M, N, K, row_scale);
    }
    return moss_launch_status();
}

}  // namespace
}  // namespace moss

using namespace moss;

MOSS_API int moss_w4g32_gemm(const void* x, const void* qw, const void* sc, const void* zp, void* y, int M, int K,
                             int N, void* stream) {
    MOSS_CHECK_ARG(x && qw && sc && zp && y && M > 0 && N > 0 && K > 0 && K % 64 == 0);
    MOSS_CHECK_ARG(MOSS_ALIGNED(x, 16) && MOSS_ALIGNED(qw, 16));
    return launch_gemm<kInt4G32>(x, qw, sc, zp, y, M, K, N, nullptr, (hipStream_t)stream);
}

namespace moss {
// FP8 e4m3 rows [N, K] with optional fp32 row scales; arguments checked by the caller.
int fp8_gemm_launch(const void* x, const void* w, const float* row_scale, void* y, int M, int K, int N,
                    hipStream_t stream) {
    return launch_gemm<kFp8E4M3>(x, w, nullptr, nullptr, y, M, K, N, row_scale, stream);
}
}  // namespace moss
