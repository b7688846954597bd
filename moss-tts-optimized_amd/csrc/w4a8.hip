// W4A8 decode mode: the reference's G32 serving arithmetic (int8 activations, integer dot
// products, fp32 group combine) on the row-packed INT4-G32 weights.
//
// Activation quantizer (src/moss_tts/_runtime/int4_dp4a.py:21-30, also fused into the
// reference's producers): per 32-value group, sc = max(RN(max|x| / 127), 1e-8),
// inv = RN(1 / sc), q = rint(x * inv) (ties to even), all in fp32 with correctly rounded
// division.  Integer sums (src/moss_tts/_runtime/dp4a_scaled.py:22-57):
// isum[n, g] = sum_k (q_w - z) * q_x, exact in int32; y[n] = sum_g f32(isum) * (s_w * s_x)
// in fp32, rounded to bf16; the paired form rounds gate and up to bf16 and applies the
// SiLU*mul epilogue (dp4a_scaled.py:64-68).
//
// Byte order of the quantized activations ("dot4 order"): within each block of 8 values,
// bytes 8b..8b+7 hold x[8b + {0, 4, 1, 5, 2, 6, 3, 7}].  That is the order in which
// (w & 0x0F0F0F0F) and ((w >> 4) & 0x0F0F0F0F) expand a row-packed code word into bytes, so
// each 8 weights cost one shift, two ands and two v_dot4_i32_i8 (unsigned codes 0..15 are
// non-negative int8).
#include "common.h"

namespace moss {
namespace {

typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));

__device__ __forceinline__ int dot4(uint32_t a, uint32_t b, int c) {
    return __builtin_amdgcn_sdot4((int)a, (int)b, c, false);
}

// One 32-lane half-wave per group of 32 (one value per lane): the group's max |x| and code
// sum are half-wave reductions, so the chain per value is short and a 12288-wide row spreads
// over 48 workgroups.  Writes the 32 int8 codes in dot4 order (value t of the group at byte
// 8 (t / 8) + dot4_slot(t % 8)), the group scale and the group's code sum (for the zero-point
// term).  Lanes past the last group load a clamped value and store nothing.
__global__ __launch_bounds__(256) void int8_quantize_g32(const uint16_t* __restrict__ x, int8_t* __restrict__ qx,
                                                         float* __restrict__ sx, int* __restrict__ qsum, int G) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    const int g = i >> 5, t = i & 31;
    const float v = bf16_bits(x[min(i, 32 * G - 1)]);
    const float sc = g32_scale(half_wave_max(fabsf(v)));
    const int q = (int)rintf(v * (1.0f / sc));
    const int sum = half_wave_sum(q);
    if (g < G) {
        qx[32 * g + 8 * (t >> 3) + dot4_slot(t & 7)] = (int8_t)q;
        if (t == 0) {
            sx[g] = sc;
            qsum[g] = sum;
        }
    }
}

// The fused normalization in front of a W4A8 projection (ACT 1: RMSNorm, ACT 2: add-RMSNorm;
// src/moss_tts/_runtime/dp4a_norm_projection.py:48-96, dp4a_fusions.py:24-61): every
// 256-thread workgroup recomputes y = bf16(bf16(s * rsqrt(mean(s^2) + eps)) * w) of the one
// K-wide row (s = x, or bf16(x + res), which workgroup 0 also stores) and its int8 groups of 32
// into LDS while its weight rows are in flight.  Thread t owns the 8-value chunks t + 256 c and
// the 4 chunks of a group sit in one DPP quad, with the summation order and rounding points of
// rmsnorm_rows<RESIDUAL, true>, so the activations are bit-identical to moss_rmsnorm_quant_g32's.
struct W8Norm {
    const uint16_t* __restrict__ x;
    const uint16_t* __restrict__ res;
    const uint16_t* __restrict__ w;
    uint16_t* __restrict__ sum_out;
    float eps;
};

// Row-per-wave GEMV: lane l owns groups l + 64 j; KG = ceil(G / 64).  QOUT (paired only):
// 32 / R waves x R rows per workgroup cover one 32-row output group, which the workgroup
// also quantizes (the down projection's activations), as the reference's fused gate/up does
// (src/moss_tts/_runtime/dp4a_scaled.py:70-78).  ACT 0 reads quantized activations; ACT 1 and
// 2 form them in the workgroup (W8Norm; K = 2048 KG).
template <int KG, int R, bool PAIRED, bool QOUT, int ACT = 0>
__global__ __launch_bounds__(QOUT ? kWave * 32 / R : 256) void w4a8_gemv_kernel(
    const uint32_t* __restrict__ qx, const float* __restrict__ sx, const int* __restrict__ qsum,
    const uint4* __restrict__ qw, const uint16_t* __restrict__ sc, const uint8_t* __restrict__ zp,
    uint16_t* __restrict__ y, uint8_t* __restrict__ oq, float* __restrict__ osx, int* __restrict__ osum, int G,
    int n_out, W8Norm nm) {
    static_assert(!QOUT || (PAIRED && (R == 2 || R == 4)), "output quantization covers 32 paired rows");
    static_assert(ACT == 0 || !QOUT, "the fused normalization runs with 256-thread workgroups");
    const int lane = threadIdx.x & (kWave - 1);
    const int wave = __builtin_amdgcn_readfirstlane(blockIdx.x * (blockDim.x / kWave) + (threadIdx.x / kWave));
    const int row0 = wave * R;
    // wave-uniform; QOUT grids hold whole groups only, and with ACT > 0 every wave takes part in
    // the workgroup's normalization first
    if (ACT == 0 && !QOUT && row0 >= n_out) return;
    constexpr int NR = PAIRED ? 2 * R : R;
    // activations first (completions are counted in order): 32 int8 per group, its scale and sum
    uint4 xa[KG], xb[KG];
    float xs[KG];
    int xq[KG];
    uint4 nx[KG], nr[KG], nw[KG];  // ACT > 0: the chunks t + 256 c of x, res and the norm weight
    if constexpr (ACT == 0) {
#pragma unroll
        for (int j = 0; j < KG; ++j) {
            const int g = lane + kWave * j;
            if (g < G) {
                const uint4* p = reinterpret_cast<const uint4*>(qx + 8 * g);
                xa[j] = p[0];
                xb[j] = p[1];
                xs[j] = sx[g];
                xq[j] = qsum[g];
            } else {
                xa[j] = xb[j] = make_uint4(0u, 0u, 0u, 0u);
                xs[j] = 0.f;
                xq[j] = 0;
            }
        }
    } else {
#pragma unroll
        for (int c = 0; c < KG; ++c) {
            const int ci = threadIdx.x + 256 * c;
            nw[c] = reinterpret_cast<const uint4*>(nm.w)[ci];
            nx[c] = reinterpret_cast<const uint4*>(nm.x)[ci];
            if constexpr (ACT == 2) nr[c] = reinterpret_cast<const uint4*>(nm.res)[ci];
        }
    }
    uint4 w[NR][KG];
    uint32_t s[NR][KG], z[NR][KG], zsh[NR][KG];  // z: the raw byte holding the zero point at bit zsh
#pragma unroll
    for (int r = 0; r < NR; ++r) {
        const int local = PAIRED ? (r % R) : r;
        const int n = min(row0 + local, n_out - 1) + ((PAIRED && r >= R) ? n_out : 0);
#pragma unroll
        for (int j = 0; j < KG; ++j) {
            const int g = lane + kWave * j;
            if (g < G) {
                const u32x4_t v = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(qw + (size_t)n * G + g));
                w[r][j] = make_uint4(v.x, v.y, v.z, v.w);
                s[r][j] = sc[(size_t)n * G + g];
                int zb;
                zero_loc(g, G, zb, zsh[r][j]);
                z[r][j] = zp[(size_t)n * (G >> 1) + zb];
            } else {
                w[r][j] = make_uint4(0u, 0u, 0u, 0u);
                s[r][j] = 0u;
                z[r][j] = 0u;
                zsh[r][j] = 0u;
            }
        }
    }
    if constexpr (ACT > 0) {
        __shared__ uint2 lq[256 * KG];
        __shared__ float lsx[64 * KG];
        __shared__ int lsum[64 * KG];
        __shared__ float red[4];
        float v[KG][8];
        float ss = 0.f;
#pragma unroll
        for (int c = 0; c < KG; ++c) {
            const int ci = threadIdx.x + 256 * c;
            uint32_t sw[4] = {nx[c].x, nx[c].y, nx[c].z, nx[c].w};
            if constexpr (ACT == 2) {
                const uint32_t bw[4] = {nr[c].x, nr[c].y, nr[c].z, nr[c].w};
#pragma unroll
                for (int p = 0; p < 4; ++p)
                    sw[p] = pack_bf16x2(bf16_lo(sw[p]) + bf16_lo(bw[p]), bf16_hi(sw[p]) + bf16_hi(bw[p]));
                if (blockIdx.x == 0) reinterpret_cast<uint4*>(nm.sum_out)[ci] = make_uint4(sw[0], sw[1], sw[2], sw[3]);
            }
#pragma unroll
            for (int p = 0; p < 4; ++p) {
                v[c][2 * p] = bf16_lo(sw[p]);
                v[c][2 * p + 1] = bf16_hi(sw[p]);
                ss = fmaf(v[c][2 * p], v[c][2 * p], ss);
                ss = fmaf(v[c][2 * p + 1], v[c][2 * p + 1], ss);
            }
        }
        ss = wave_sum(ss);
        if (lane == 0) red[threadIdx.x / kWave] = ss;
        __syncthreads();
        float total = 0.f;
#pragma unroll
        for (int i = 0; i < 4; ++i) total += red[i];
        const float inv = rsqrtf(total / (float)(32 * G) + nm.eps);
#pragma unroll
        for (int c = 0; c < KG; ++c) {
            const int ci = threadIdx.x + 256 * c;
            const uint32_t wv[4] = {nw[c].x, nw[c].y, nw[c].z, nw[c].w};
            float yv[8];
#pragma unroll
            for (int p = 0; p < 4; ++p) {
                const float a = round_bf16(v[c][2 * p] * inv) * bf16_lo(wv[p]);
                const float b = round_bf16(v[c][2 * p + 1] * inv) * bf16_hi(wv[p]);
                const uint32_t o = pack_bf16x2(a, b);
                yv[2 * p] = bf16_lo(o);
                yv[2 * p + 1] = bf16_hi(o);
            }
            float m = 0.f;
#pragma unroll
            for (int i = 0; i < 8; ++i) m = fmaxf(m, fabsf(yv[i]));
            const float scale = g32_scale(quad_max(m));
            uint32_t lo, hi;
            const int part = quantize8_dot4(yv, 1.0f / scale, lo, hi);
            const float gsum = quad_sum((float)part);  // |sum| <= 32 * 127: exact in fp32
            lq[ci] = make_uint2(lo, hi);
            if ((ci & 3) == 0) {
                lsx[ci / 4] = scale;
                lsum[ci / 4] = (int)gsum;
            }
        }
        __syncthreads();
        if (row0 >= n_out) return;  // after the workgroup's barriers
#pragma unroll
        for (int j = 0; j < KG; ++j) {
            const int g = lane + kWave * j;
            const uint4* p = reinterpret_cast<const uint4*>(lq) + 2 * g;
            xa[j] = p[0];
            xb[j] = p[1];
            xs[j] = lsx[g];
            xq[j] = lsum[g];
        }
    }
    uint32_t mask = 0x0F0F0F0Fu;
    asm volatile("" : "+v"(mask));
    float out[NR];
#pragma unroll
    for (int r = 0; r < NR; ++r) {
        float part = 0.f;
#pragma unroll
        for (int j = 0; j < KG; ++j) {
            const uint32_t words[4] = {w[r][j].x, w[r][j].y, w[r][j].z, w[r][j].w};
            const uint32_t xw[8] = {xa[j].x, xa[j].y, xa[j].z, xa[j].w, xb[j].x, xb[j].y, xb[j].z, xb[j].w};
            int isum = -(int)((z[r][j] >> zsh[r][j]) & 15u) * xq[j];
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                isum = dot4(words[c] & mask, xw[2 * c], isum);
                isum = dot4((words[c] >> 4) & mask, xw[2 * c + 1], isum);
            }
            part = fmaf((float)isum, bf16_bits((uint16_t)s[r][j]) * xs[j], part);
        }
        out[r] = wave_sum(part);
    }
    uint16_t val[R];
#pragma unroll
    for (int r = 0; r < R; ++r) val[r] = PAIRED ? silu_mul_rounded_bits(out[r], out[R + r]) : f32_to_bf16(out[r]);
    if (lane == 0) {
#pragma unroll
        for (int r = 0; r < R; ++r)
            if (row0 + r < n_out) y[row0 + r] = val[r];
    }
    if constexpr (QOUT) {
        // rows 32 b .. 32 b + 31 of this workgroup form output group b
        __shared__ float grp[32];
        const int wl = threadIdx.x / kWave;
        if (lane == 0) {
#pragma unroll
            for (int r = 0; r < R; ++r) grp[R * wl + r] = bf16_bits(val[r]);
        }
        __syncthreads();
        if (wl == 0) {
            const int b = blockIdx.x;
            const float v = lane < 32 ? grp[lane] : 0.f;
            const float scale = g32_scale(wave_max(fabsf(v)));
            const float q = rintf(v * (1.0f / scale));
            const float total = wave_sum(q);  // |sum| <= 32 * 127: exact in fp32
            if (lane < 32) oq[32 * b + 8 * (lane >> 3) + dot4_slot(lane & 7)] = (uint8_t)(int)q;
            if (lane == 0) {
                osx[b] = scale;
                osum[b] = (int)total;
            }
        }
    }
}

template <bool PAIRED, bool QOUT>
int launch_w4a8(const void* qx, const void* sx, const void* qsum, const void* qw, const void* sc, const void* zp,
                void* y, void* oq, void* osx, void* osum, int K, int n_out, int rows, hipStream_t st) {
    const int G = K / 32, KG = (G + kWave - 1) / kWave;
    if (rows == 0) rows = QOUT ? 2 : 1;
    if (QOUT && rows == 1) return (int)hipErrorInvalidValue;
    const int waves = (n_out + rows - 1) / rows;
    const int wpb = QOUT ? 32 / rows : 4;
    const dim3 grid((waves + wpb - 1) / wpb), block(kWave * wpb);
#define MOSS_W4A8(KGV, RV)                                                                                        \
    if (KG == KGV && rows == RV) {                                                                                \
        hipLaunchKernelGGL((w4a8_gemv_kernel<KGV, RV, PAIRED, QOUT && RV != 1>), grid, block, 0, st,              \
                           (const uint32_t*)qx, (const float*)sx, (const int*)qsum, (const uint4*)qw,             \
                           (const uint16_t*)sc, (const uint8_t*)zp, (uint16_t*)y, (uint8_t*)oq, (float*)osx,      \
                           (int*)osum, G, n_out, W8Norm{});                                                       \
        return moss_launch_status();                                                                              \
    }
#define MOSS_W4A8_R(KGV) MOSS_W4A8(KGV, 1) MOSS_W4A8(KGV, 2) MOSS_W4A8(KGV, 4)
    MOSS_W4A8_R(1) MOSS_W4A8_R(2) MOSS_W4A8_R(3) MOSS_W4A8_R(4) MOSS_W4A8_R(5) MOSS_W4A8_R(6) MOSS_W4A8_R(7)
    MOSS_W4A8_R(8)
#undef MOSS_W4A8_R
#undef MOSS_W4A8
    return (int)hipErrorInvalidValue;
}

// K = 2048 KG, KG in {1, 2, 4} (K = 2048, 4096, 8192).
template <bool PAIRED>
int launch_w4a8_norm(const W8Norm& nm, const void* qw, const void* sc, const void* zp, void* y, int K, int n_out,
                     int rows, hipStream_t st) {
    const int G = K / 32, KG = K / 2048;
    if (rows == 0) rows = 1;
    const int waves = (n_out + rows - 1) / rows;
    const dim3 grid((waves + 3) / 4), block(256);
#define MOSS_W4A8N(KGV, RV, ACTV)                                                                                 \
    if (KG == KGV && rows == RV) {                                                                                \
        hipLaunchKernelGGL((w4a8_gemv_kernel<KGV, RV, PAIRED, false, ACTV>), grid, block, 0, st, nullptr,         \
                           nullptr, nullptr, (const uint4*)qw, (const uint16_t*)sc, (const uint8_t*)zp,           \
                           (uint16_t*)y, nullptr, nullptr, nullptr, G, n_out, nm);                                \
        return moss_launch_status();                                                                              \
    }
#define MOSS_W4A8N_R(KGV, ACTV) MOSS_W4A8N(KGV, 1, ACTV) MOSS_W4A8N(KGV, 2, ACTV) MOSS_W4A8N(KGV, 4, ACTV)
    if (nm.res) {
        MOSS_W4A8N_R(1, 2) MOSS_W4A8N_R(2, 2) MOSS_W4A8N_R(4, 2)
    } else {
        MOSS_W4A8N_R(1, 1) MOSS_W4A8N_R(2, 1) MOSS_W4A8N_R(4, 1)
    }
#undef MOSS_W4A8N_R
#undef MOSS_W4A8N
    return (int)hipErrorInvalidValue;
}

}  // namespace
}  // namespace moss

using namespace moss;

MOSS_API int moss_int8_quantize_g32(const void* x, void* qx, void* sx, void* qsum, int K, void* stream) {
    MOSS_CHECK_ARG(x && qx && sx && qsum && K > 0 && K % 32 == 0);
    MOSS_CHECK_ARG(MOSS_ALIGNED(x, 16) && MOSS_ALIGNED(qx, 16) && MOSS_ALIGNED(sx, 4) && MOSS_ALIGNED(qsum, 4));
    const int G = K / 32;
    hipLaunchKernelGGL(int8_quantize_g32, dim3((32 * G + 255) / 256), dim3(256), 0, (hipStream_t)stream,
                       (const uint16_t*)x, (int8_t*)qx, (float*)sx, (int*)qsum, G);
    return moss_launch_status();
}

static int check_w4a8(const void* qx, const void* sx, const void* qsum, const void* qw, const void* sc, const void* zp,
                      const void* y, int K, int rows) {
    MOSS_CHECK_ARG(qx && sx && qsum && qw && sc && zp && y && K > 0 && K % 64 == 0 && K <= 16384);
    MOSS_CHECK_ARG(rows == 0 || rows == 1 || rows == 2 || rows == 4);
    MOSS_CHECK_ARG(MOSS_ALIGNED(qx, 16) && MOSS_ALIGNED(qw, 16));
    return 0;
}

MOSS_API int moss_w4a8_gemv(const void* qx, const void* sx, const void* qsum, const void* qw, const void* sc,
                            const void* zp, void* y, int K, int N, int rows_per_wave, void* stream) {
    if (int rc = check_w4a8(qx, sx, qsum, qw, sc, zp, y, K, rows_per_wave)) return rc;
    MOSS_CHECK_ARG(N > 0);
    return launch_w4a8<false, false>(qx, sx, qsum, qw, sc, zp, y, nullptr, nullptr, nullptr, K, N, rows_per_wave,
                                     (hipStream_t)stream);
}

MOSS_API int moss_w4a8_gateup_silu(const void* qx, const void* sx, const void* qsum, const void* qw, const void* sc,
                                   const void* zp, void* y, void* out_qx, void* out_sx, void* out_qsum, int K,
                                   int N_half, int rows_per_wave, void* stream) {
    if (int rc = check_w4a8(qx, sx, qsum, qw, sc, zp, y, K, rows_per_wave)) return rc;
    MOSS_CHECK_ARG(N_half > 0);
    const bool quant = out_qx != nullptr;
    MOSS_CHECK_ARG(quant == (out_sx != nullptr) && quant == (out_qsum != nullptr));
    if (!quant)
        return launch_w4a8<true, false>(qx, sx, qsum, qw, sc, zp, y, nullptr, nullptr, nullptr, K, N_half,
                                        rows_per_wave, (hipStream_t)stream);
    MOSS_CHECK_ARG(N_half % 32 == 0 && rows_per_wave != 1);
    MOSS_CHECK_ARG(MOSS_ALIGNED(out_sx, 4) && MOSS_ALIGNED(out_qsum, 4));
    return launch_w4a8<true, true>(qx, sx, qsum, qw, sc, zp, y, out_qx, out_sx, out_qsum, K, N_half,
                                   rows_per_wave, (hipStream_t)stream);
}

static int w4a8_norm_entry(bool paired, const void* x, const void* res, const void* norm_w, void* sum_out, float eps,
                           const void* qw, const void* sc, const void* zp, void* y, int K, int n_out,
                           int rows_per_wave, void* stream) {
    if (int rc = moss_check_norm_args(x, res, norm_w, sum_out, K, eps)) return rc;
    MOSS_CHECK_ARG(qw && sc && zp && y && n_out > 0);
    MOSS_CHECK_ARG(K == 2048 || K == 4096 || K == 8192);
    MOSS_CHECK_ARG(rows_per_wave == 0 || rows_per_wave == 1 || rows_per_wave == 2 || rows_per_wave == 4);
    MOSS_CHECK_ARG(MOSS_ALIGNED(qw, 16));
    const W8Norm nm{(const uint16_t*)x, (const uint16_t*)res, (const uint16_t*)norm_w, (uint16_t*)sum_out, eps};
    return paired ? launch_w4a8_norm<true>(nm, qw, sc, zp, y, K, n_out, rows_per_wave, (hipStream_t)stream)
                  : launch_w4a8_norm<false>(nm, qw, sc, zp, y, K, n_out, rows_per_wave, (hipStream_t)stream);
}

MOSS_API int moss_w4a8_norm_gemv(const void* x, const void* res, const void* norm_w, void* sum_out, float eps,
                                 const void* qw, const void* sc, const void* zp, void* y, int K, int N,
                                 int rows_per_wave, void* stream) {
    return w4a8_norm_entry(false, x, res, norm_w, sum_out, eps, qw, sc, zp, y, K, N, rows_per_wave, stream);
}

MOSS_API int moss_w4a8_norm_gateup_silu(const void* x, const void* res, const void* norm_w, void* sum_out, float eps,
                                        const void* qw, const void* sc, const void* zp, void* y, int K, int N_half,
                                        int rows_per_wave, void* stream) {
    return w4a8_norm_entry(true, x, res, norm_w, sum_out, eps, qw, sc, zp, y, K, N_half, rows_per_wave, stream);
}
