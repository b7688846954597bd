// (add+)RMSNorm fused in front of a decode projection: every workgroup recomputes the normalized
// 4096-wide (2048 * CH) row into LDS while its weight loads are in flight.
#pragma once

#include "common.h"

namespace moss {

// Fused normalization in front of the projection (the reference's fused add+RMSNorm+projection,
// src/moss_tts/_runtime/dp4a_norm_projection.py:48-96, with the rounding points of
// src/moss_tts/_runtime/kernels.py:50-90):
//   NORM 1: xn = bf16(bf16(x * rsqrt(mean(x^2) + eps)) * w)
//   NORM 2: s = bf16(x + res), xn = the same on s; workgroup 0 also stores s to sum_out.
// Every workgroup (256 threads) recomputes it from the 8 KB row (an L2 hit) into LDS while its
// weight loads are in flight; thread t owns 8-value chunks t + 256 c, c < K / 2048, exactly
// as rmsnorm_rows does, so the normalized row is bit-identical to moss_rmsnorm's.
struct NormArgs {
    const uint16_t* __restrict__ res;
    const uint16_t* __restrict__ w;
    uint16_t* __restrict__ sum_out;
    float eps;
};

template <int CH>
struct NormLoad {
    uint4 x[CH], r[CH], w[CH];
};

// Issued before the weight-row loads: vector-memory completions are counted in order, so the
// normalization below then waits only for these and overlaps the weight stream.
template <int NORM, int CH>
__device__ __forceinline__ void norm_load(NormLoad<CH>& nl, const uint16_t* __restrict__ x, const NormArgs& na) {
    const int t = threadIdx.x;
#pragma unroll
    for (int c = 0; c < CH; ++c) {
        const int ci = t + 256 * c;
        nl.x[c] = reinterpret_cast<const uint4*>(x)[ci];
        if constexpr (NORM == 2) nl.r[c] = reinterpret_cast<const uint4*>(na.res)[ci];
        nl.w[c] = reinterpret_cast<const uint4*>(na.w)[ci];
    }
}

template <int NORM, int CH>
__device__ __forceinline__ void norm_into_lds(const NormLoad<CH>& nl, const NormArgs& na, uint16_t* xn, float* red,
                                              int K) {
    const int t = threadIdx.x;
    uint32_t pk[CH][4];  // the row as packed bf16 pairs between the two phases (8 VGPRs, not 16)
    float ss = 0.f;
#pragma unroll
    for (int c = 0; c < CH; ++c) {
        const int ci = t + 256 * c;
        uint32_t sw[4] = {nl.x[c].x, nl.x[c].y, nl.x[c].z, nl.x[c].w};
        if constexpr (NORM == 2) {
            const uint32_t bw[4] = {nl.r[c].x, nl.r[c].y, nl.r[c].z, nl.r[c].w};
#pragma unroll
            for (int p = 0; p < 4; ++p) {
                sw[p] = pack_bf16x2(bf16_lo(sw[p]) + bf16_lo(bw[p]),
                            bf16_hi(sw[p]) + bf16_hi(bw[p]));
            }
            if (blockIdx.x == 0)
                reinterpret_cast<uint4*>(na.sum_out)[ci] = make_uint4(sw[0], sw[1], sw[2], sw[3]);
        }
#pragma unroll
        for (int p = 0; p < 4; ++p) {
            pk[c][p] = sw[p];
            const float lo = bf16_lo(sw[p]), hi = bf16_hi(sw[p]);
            ss = fmaf(lo, lo, ss);
            ss = fmaf(hi, hi, ss);
        }
    }
    ss = wave_sum(ss);
    if ((t & (kWave - 1)) == 0) red[t / kWave] = ss;
    __syncthreads();
    const float inv = rsqrtf((((red[0] + red[1]) + red[2]) + red[3]) / (float)K + na.eps);
#pragma unroll
    for (int c = 0; c < CH; ++c) {
        const int ci = t + 256 * c;
        const uint32_t wv[4] = {nl.w[c].x, nl.w[c].y, nl.w[c].z, nl.w[c].w};
        uint32_t o[4];
#pragma unroll
        for (int p = 0; p < 4; ++p) {
            const float a = round_bf16(bf16_lo(pk[c][p]) * inv) * bf16_lo(wv[p]);
            const float b = round_bf16(bf16_hi(pk[c][p]) * inv) * bf16_hi(wv[p]);
            o[p] = pack_bf16x2(a, b);
        }
        reinterpret_cast<uint4*>(xn)[ci] = make_uint4(o[0], o[1], o[2], o[3]);
    }
    __syncthreads();
}

}  // namespace moss
