// RMSNorm / add-RMSNorm, q/k head-norm + RoPE + KV-cache write, and the standalone SiLU*mul.
//
// Rounding points follow the reference kernels:
//   rmsnorm       y = bf16(bf16(x * rsqrt(mean(x^2) + eps)) * w)        src/moss_tts/_runtime/kernels.py:50-59
//   add_rmsnorm   s = bf16(x + r); y = rmsnorm(s)                        src/moss_tts/_runtime/kernels.py:69-82
//   qk-norm+RoPE  xn = bf16(bf16(x*r) * w[d]); out = bf16(bf16(xn*cos) + bf16(+-xs*sin))
//                 with xs the value at (d+64)%128 and float negation for d < 64
//                 src/moss_tts/_runtime/kernels.py:142-170, prefill_qkv.py:7-28
//   silu_mul      y = bf16(bf16(g / (1 + exp(-g))) * u)                  src/moss_tts/_runtime/prefill_pointwise.py:18-31
#include "common.h"

namespace moss {
namespace {

constexpr int kNormThreads = 256;

__device__ __forceinline__ float block_sum(float v, float* lds) {
    v = wave_sum(v);
    const int w = threadIdx.x / kWave;
    if ((threadIdx.x & (kWave - 1)) == 0) lds[w] = v;
    __syncthreads();
    float s = 0.f;
#pragma unroll
    for (int i = 0; i < kNormThreads / kWave; ++i) s += lds[i];
    return s;
}

// One workgroup per row; each thread owns 8-value chunks c = tid, tid + 256, ...
// (n % 8 == 0, n <= 8 * 256 * kMaxChunks).
constexpr int kMaxChunks = 4;

// QUANT: also quantize y per group of 32 to int8 (dot4 order, see common.h) with fp32 group
// scales and code sums, as the reference's fused norm + quantizer does
// (src/moss_tts/_runtime/dp4a_fusions.py:24-40); y may then be null.  A group's 4 chunks
// belong to the 4 lanes of one DPP quad.
// PARTS: x is not read; each value is formed from S fp32 partial sums of a split-K GEMM,
// parts[z][row][col] added in z order from 0 and rounded to bf16 -- exactly what gemm_reduce
// (w4g32_gemm.hip) writes -- so reduce-then-norm takes one launch and no bf16 round trip.
// The body carries no aliasing promises; the kernels below state them.
template <bool RESIDUAL, bool QUANT, bool PARTS>
__device__ __forceinline__ void rmsnorm_row_body(const uint16_t* x, const uint16_t* res, const uint16_t* w,
                                                 uint16_t* sum_out, uint16_t* y, int n, float eps, uint2* qx,
                                                 float* sx, int* qsum, const float* parts, int S) {
    __shared__ float lds[kNormThreads / kWave];
    const size_t row = blockIdx.x;
    const int chunks = n / 8;
    const uint4* xr = reinterpret_cast<const uint4*>(x + row * n);
    const uint4* rr = reinterpret_cast<const uint4*>(res + row * n);
    float v[kMaxChunks][8];
    float ss = 0.f;
    // the weight loads go out first so they overlap the reduction
    const uint4* wr = reinterpret_cast<const uint4*>(w);
    uint4 wv4[kMaxChunks];
#pragma unroll
    for (int c = 0; c < kMaxChunks; ++c) {
        const int ci = threadIdx.x + c * kNormThreads;
        wv4[c] = ci < chunks ? wr[ci] : make_uint4(0u, 0u, 0u, 0u);
    }
#pragma unroll
    for (int c = 0; c < kMaxChunks; ++c) {
        const int ci = threadIdx.x + c * kNormThreads;
        if (ci < chunks) {
            uint4 a;
            if constexpr (PARTS) {
                const size_t mn = (size_t)gridDim.x * n;
                const float* pr = parts + row * n + 8 * ci;
                float acc[8];
#pragma unroll
                for (int k = 0; k < 8; ++k) acc[k] = 0.f;
                if (S <= 2) {
                    for (int z = 0; z < S; ++z) {
                        const float4 p0 = reinterpret_cast<const float4*>(pr + z * mn)[0];
                        const float4 p1 = reinterpret_cast<const float4*>(pr + z * mn)[1];
                        acc[0] += p0.x, acc[1] += p0.y, acc[2] += p0.z, acc[3] += p0.w;
                        acc[4] += p1.x, acc[5] += p1.y, acc[6] += p1.z, acc[7] += p1.w;
                    }
                } else {
                    // deeper splits (short prompts): 4 partials loaded before they are added, so the
                    // loads of a row do not wait on each other; the same split-order sum
                    for (int z0 = 0; z0 < S; z0 += 4) {
                        float4 p[4][2];
#pragma unroll
                        for (int z = 0; z < 4; ++z)
                            if (z0 + z < S) {
                                p[z][0] = reinterpret_cast<const float4*>(pr + (z0 + z) * mn)[0];
                                p[z][1] = reinterpret_cast<const float4*>(pr + (z0 + z) * mn)[1];
                            }
#pragma unroll
                        for (int z = 0; z < 4; ++z)
                            if (z0 + z < S) {
                                acc[0] += p[z][0].x, acc[1] += p[z][0].y, acc[2] += p[z][0].z, acc[3] += p[z][0].w;
                                acc[4] += p[z][1].x, acc[5] += p[z][1].y, acc[6] += p[z][1].z, acc[7] += p[z][1].w;
                            }
                    }
                }
                a = make_uint4(pack_bf16x2(acc[0], acc[1]), pack_bf16x2(acc[2], acc[3]), pack_bf16x2(acc[4], acc[5]),
                               pack_bf16x2(acc[6], acc[7]));
            } else {
                a = xr[ci];
            }
            const uint32_t aw[4] = {a.x, a.y, a.z, a.w};
            uint32_t sw[4];
            if constexpr (RESIDUAL) {
                const uint4 b = rr[ci];
                const uint32_t bw[4] = {b.x, b.y, b.z, b.w};
#pragma unroll
                for (int p = 0; p < 4; ++p) {
                    sw[p] = pack_bf16x2(bf16_lo(aw[p]) + bf16_lo(bw[p]),
                                bf16_hi(aw[p]) + bf16_hi(bw[p]));
                }
                reinterpret_cast<uint4*>(sum_out + row * n)[ci] = make_uint4(sw[0], sw[1], sw[2], sw[3]);
            } else {
#pragma unroll
                for (int p = 0; p < 4; ++p) sw[p] = aw[p];
            }
#pragma unroll
            for (int p = 0; p < 4; ++p) {
                v[c][2 * p] = bf16_lo(sw[p]);
                v[c][2 * p + 1] = bf16_hi(sw[p]);
                ss = fmaf(v[c][2 * p], v[c][2 * p], ss);
                ss = fmaf(v[c][2 * p + 1], v[c][2 * p + 1], ss);
            }
        }
    }
    const float inv = rsqrtf(block_sum(ss, lds) / (float)n + eps);
#pragma unroll
    for (int c = 0; c < kMaxChunks; ++c) {
        const int ci = threadIdx.x + c * kNormThreads;
        if (c * kNormThreads >= chunks) break;  // block-uniform
        float yv[8];
        const bool active = ci < chunks;
        if (active) {
            const uint4 ww = wv4[c];
            const uint32_t wv[4] = {ww.x, ww.y, ww.z, ww.w};
            uint32_t o[4];
#pragma unroll
            for (int p = 0; p < 4; ++p) {
                const float a = round_bf16(v[c][2 * p] * inv) * bf16_lo(wv[p]);
                const float b = round_bf16(v[c][2 * p + 1] * inv) * bf16_hi(wv[p]);
                o[p] = pack_bf16x2(a, b);
                yv[2 * p] = bf16_lo(o[p]);
                yv[2 * p + 1] = bf16_hi(o[p]);
            }
            if (!QUANT || y) reinterpret_cast<uint4*>(y + row * n)[ci] = make_uint4(o[0], o[1], o[2], o[3]);
        } else {
#pragma unroll
            for (int i = 0; i < 8; ++i) yv[i] = 0.f;
        }
        if constexpr (QUANT) {
            float m = 0.f;
#pragma unroll
            for (int i = 0; i < 8; ++i) m = fmaxf(m, fabsf(yv[i]));
            const float scale = g32_scale(quad_max(m));
            uint32_t lo, hi;
            const int part = quantize8_dot4(yv, 1.0f / scale, lo, hi);
            const float total = quad_sum((float)part);  // |sum| <= 32 * 127: exact in fp32
            if (active) {
                qx[row * chunks + ci] = make_uint2(lo, hi);
                if ((ci & 3) == 0) {
                    sx[row * (n / 32) + ci / 4] = scale;
                    qsum[row * (n / 32) + ci / 4] = (int)total;
                }
            }
        }
    }
}

template <bool RESIDUAL, bool QUANT = false, bool PARTS = false>
__global__ __launch_bounds__(kNormThreads) void rmsnorm_rows(const uint16_t* __restrict__ x,
                                                             const uint16_t* __restrict__ res,
                                                             const uint16_t* __restrict__ w,
                                                             uint16_t* __restrict__ sum_out,
                                                             uint16_t* __restrict__ y, int n, float eps,
                                                             uint2* __restrict__ qx = nullptr,
                                                             float* __restrict__ sx = nullptr,
                                                             int* __restrict__ qsum = nullptr,
                                                             const float* __restrict__ parts = nullptr, int S = 0) {
    rmsnorm_row_body<RESIDUAL, QUANT, PARTS>(x, res, w, sum_out, y, n, eps, qx, sx, qsum, parts, S);
}

// add-RMSNorm with sum_out == x allowed (x and sum_out carry no __restrict__): each thread reads
// its chunks of x before it writes the same chunks of sum_out, and no thread touches another's.
__global__ __launch_bounds__(kNormThreads) void add_rmsnorm_rows_inplace(const uint16_t* x,
                                                                         const uint16_t* __restrict__ res,
                                                                         const uint16_t* __restrict__ w,
                                                                         uint16_t* sum_out,
                                                                         uint16_t* __restrict__ y, int n, float eps) {
    rmsnorm_row_body<true, false, false>(x, res, w, sum_out, y, n, eps, nullptr, nullptr, nullptr, nullptr, 0);
}

// One wave per (token, head); lane l owns dims l and l + 64, which are each other's RoPE
// partners, so only the sum of squares crosses lanes.  Heads 0..31 are queries, 32..39 keys.
__global__ __launch_bounds__(256) void qk_norm_rope_kv(const uint16_t* __restrict__ qkv,
                                                       const uint16_t* __restrict__ qw,
                                                       const uint16_t* __restrict__ kw,
                                                       const uint16_t* __restrict__ cos_t,
                                                       const uint16_t* __restrict__ sin_t,
                                                       uint16_t* __restrict__ q_out, uint16_t* __restrict__ kc,
                                                       uint16_t* __restrict__ vc, const int64_t* __restrict__ pos,
                                                       int L, int ntok, float eps, int cos_by_position) {
    constexpr int QH = 32, KH = 8, D = 128, ROW = (QH + 2 * KH) * D;  // 6144
    const int wave = blockIdx.x * 4 + threadIdx.x / kWave;
    if (wave >= ntok * (QH + KH)) return;
    const int t = wave / (QH + KH), h = wave % (QH + KH);
    const int l = threadIdx.x & (kWave - 1);
    const bool is_q = h < QH;
    const size_t base = (size_t)t * ROW + (is_q ? h * D : QH * D + (h - QH) * D);
    const uint16_t* wt = is_q ? qw : kw;
    const float a = bf16_bits(qkv[base + l]);       // dim l
    const float b = bf16_bits(qkv[base + l + 64]);  // dim l + 64
    // positions live on the device (no host check without a sync): one outside [0, L) is clamped,
    // so a bad position writes row 0 or L-1 instead of touching memory outside the cache
    const int64_t p = min(max(pos[t], (int64_t)0), (int64_t)(L - 1));
    const size_t crow = cos_by_position ? (size_t)p : (size_t)t;  // table row: by position or token
    const float c0 = bf16_bits(cos_t[crow * D + l]), c1 = bf16_bits(cos_t[crow * D + l + 64]);
    const float s0 = bf16_bits(sin_t[crow * D + l]), s1 = bf16_bits(sin_t[crow * D + l + 64]);
    uint16_t o0, o1;
    head_norm_rope(a, b, bf16_bits(wt[l]), bf16_bits(wt[l + 64]), c0, c1, s0, s1, eps, o0, o1);
    if (is_q) {
        uint16_t* dst = q_out + ((size_t)t * QH + h) * D;
        dst[l] = o0;
        dst[l + 64] = o1;
    } else {
        const int kh = h - QH;
        uint16_t* kd = kc + ((size_t)kh * L + p) * D;
        uint16_t* vd = vc + ((size_t)kh * L + p) * D;
        kd[l] = o0;
        kd[l + 64] = o1;
        const size_t vb = (size_t)t * ROW + (QH + KH) * D + kh * D;
        vd[l] = qkv[vb + l];
        vd[l + 64] = qkv[vb + l + 64];
    }
}

// The same with 16 lanes per head and four heads per wave (head4_norm_rope): lane j of a head holds
// dims 4 j .. + 3 and their RoPE partners 64 + 4 j .. + 3, moved with 8-byte loads and stores; every
// output equals qk_norm_rope_kv's bit for bit.  Requires 8-byte aligned rows (checked by the caller).
// PARTS: the QKV rows are a K-split GEMM's S fp32 partials [S, ntok, 6144] (16-byte aligned), summed
// in split order and rounded to bf16 as gemm_reduce does, so the outputs equal gemm_reduce followed
// by the plain form bit for bit.
template <bool PARTS = false>
__global__ __launch_bounds__(256) void qk_norm_rope_kv4(const uint16_t* __restrict__ qkv,
                                                        const uint16_t* __restrict__ qw,
                                                        const uint16_t* __restrict__ kw,
                                                        const uint16_t* __restrict__ cos_t,
                                                        const uint16_t* __restrict__ sin_t,
                                                        uint16_t* __restrict__ q_out, uint16_t* __restrict__ kc,
                                                        uint16_t* __restrict__ vc, const int64_t* __restrict__ pos,
                                                        int L, int ntok, float eps, int cos_by_position,
                                                        const float* __restrict__ parts = nullptr, int S = 0) {
    constexpr int QH = 32, KH = 8, D = 128, ROW = (QH + 2 * KH) * D;  // 6144
    const int g = (int)((blockIdx.x * blockDim.x + threadIdx.x) >> 4);  // (token, head); 16-lane aligned
    if (g >= ntok * (QH + KH)) return;                                    // whole 16-lane groups only
    const int t = g / (QH + KH), h = g % (QH + KH), j = threadIdx.x & 15;
    const bool is_q = h < QH;
    const size_t base = (size_t)t * ROW + (is_q ? h * D : QH * D + (h - QH) * D);
    const uint16_t* wt = is_q ? qw : kw;
    auto ld4 = [](const uint16_t* p) { return *reinterpret_cast<const uint2*>(p); };
    auto row4 = [&](size_t off) {  // QKV elements off .. off + 3
        if constexpr (PARTS) {
            // partials loaded 8 at a time before they are added, in split order
            float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
            for (int z0 = 0; z0 < S; z0 += 8) {
                float4 v[8];
#pragma unroll
                for (int z = 0; z < 8; ++z)
                    if (z0 + z < S) v[z] = *reinterpret_cast<const float4*>(parts + (size_t)(z0 + z) * ntok * ROW + off);
#pragma unroll
                for (int z = 0; z < 8; ++z)
                    if (z0 + z < S) {
                        acc.x += v[z].x;
                        acc.y += v[z].y;
                        acc.z += v[z].z;
                        acc.w += v[z].w;
                    }
            }
            return make_uint2(pack_bf16x2(acc.x, acc.y), pack_bf16x2(acc.z, acc.w));
        } else {
            return ld4(qkv + off);
        }
    };
    const uint2 xa = row4(base + 4 * j), xb = row4(base + 64 + 4 * j);
    const int64_t p = min(max(pos[t], (int64_t)0), (int64_t)(L - 1));
    const size_t crow = cos_by_position ? (size_t)p : (size_t)t;
    uint2 lo, hi;
    head4_norm_rope(xa, xb, ld4(wt + 4 * j), ld4(wt + 64 + 4 * j), ld4(cos_t + crow * D + 4 * j),
                    ld4(cos_t + crow * D + 64 + 4 * j), ld4(sin_t + crow * D + 4 * j), ld4(sin_t + crow * D + 64 + 4 * j),
                    eps, lo, hi);
    if (is_q) {
        uint16_t* dst = q_out + ((size_t)t * QH + h) * D;
        *reinterpret_cast<uint2*>(dst + 4 * j) = lo;
        *reinterpret_cast<uint2*>(dst + 64 + 4 * j) = hi;
    } else {
        const int kh = h - QH;
        uint16_t* kd = kc + ((size_t)kh * L + p) * D;
        uint16_t* vd = vc + ((size_t)kh * L + p) * D;
        *reinterpret_cast<uint2*>(kd + 4 * j) = lo;
        *reinterpret_cast<uint2*>(kd + 64 + 4 * j) = hi;
        const size_t vb = (size_t)t * ROW + (QH + KH) * D + kh * D;
        *reinterpret_cast<uint2*>(vd + 4 * j) = row4(vb + 4 * j);
        *reinterpret_cast<uint2*>(vd + 64 + 4 * j) = row4(vb + 64 + 4 * j);
    }
}

// x [rows, 2n] (gate | up) -> y [rows, n]; n % 2 == 0.
__global__ __launch_bounds__(256) void silu_mul_rows(const uint32_t* __restrict__ x, uint32_t* __restrict__ y,
                                                     int n, size_t pairs) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= pairs) return;
    const size_t half = (size_t)n / 2;
    const size_t row = i / half, c = i % half;
    const uint32_t g = x[row * n + c];         // gate pair (row, 2c..2c+1)
    const uint32_t u = x[row * n + half + c];  // up pair
    float r[2];
#pragma unroll
    for (int p = 0; p < 2; ++p) {
        const float gv = p ? bf16_hi(g) : bf16_lo(g);
        const float uv = p ? bf16_hi(u) : bf16_lo(u);
        r[p] = silu_mul_bf16(gv, uv);
    }
    y[row * half + c] = pack_bf16x2(r[0], r[1]);
}

}  // namespace

// The split-K reduction of a GEMM's fp32 partials fused with the residual add and RMSNorm that
// follow it (rows x n outputs, S partials each; n % 8 == 0, 16-byte aligned buffers).
int qk_rope_from_parts(const float* parts, int S, const void* q_weight, const void* k_weight, const void* cos,
                       const void* sin, void* q_out, void* k_cache, void* v_cache, const void* positions, int L,
                       int ntok, float eps, hipStream_t st) {
    if (S < 1) return (int)hipErrorInvalidValue;
    const int waves = ntok * 40;
    hipLaunchKernelGGL(qk_norm_rope_kv4<true>, dim3((waves + 15) / 16), dim3(256), 0, st, (const uint16_t*)nullptr,
                       (const uint16_t*)q_weight, (const uint16_t*)k_weight, (const uint16_t*)cos, (const uint16_t*)sin,
                       (uint16_t*)q_out, (uint16_t*)k_cache, (uint16_t*)v_cache, (const int64_t*)positions, L, ntok,
                       eps, 1, parts, S);
    return moss_launch_status();
}

int add_rmsnorm_inplace(void* xs, const void* res, const void* w, void* y, int rows, int n, float eps, hipStream_t st) {
    hipLaunchKernelGGL(add_rmsnorm_rows_inplace, dim3(rows), dim3(kNormThreads), 0, st, (const uint16_t*)xs,
                       (const uint16_t*)res, (const uint16_t*)w, (uint16_t*)xs, (uint16_t*)y, n, eps);
    return moss_launch_status();
}

int addnorm_from_parts(const float* parts, int S, const void* res, const void* w, void* sum_out, void* y, int rows,
                       int n, float eps, hipStream_t st) {
    hipLaunchKernelGGL((rmsnorm_rows<true, false, true>), dim3(rows), dim3(kNormThreads), 0, st,
                       (const uint16_t*)nullptr, (const uint16_t*)res, (const uint16_t*)w, (uint16_t*)sum_out,
                       (uint16_t*)y, n, eps, (uint2*)nullptr, (float*)nullptr, (int*)nullptr, parts, S);
    return moss_launch_status();
}

}  // namespace moss

using namespace moss;

MOSS_API int moss_rmsnorm(const void* x, const void* res, const void* w, void* sum_out, void* y, int rows, int n,
                          float eps, void* stream) {
    MOSS_CHECK_ARG(x && w && y && rows > 0 && n > 0 && n % 8 == 0 && n <= 8 * kNormThreads * kMaxChunks);
    MOSS_CHECK_ARG(MOSS_ALIGNED(x, 16) && MOSS_ALIGNED(w, 16) && MOSS_ALIGNED(y, 16));
    MOSS_CHECK_ARG(!res || (sum_out && MOSS_ALIGNED(res, 16) && MOSS_ALIGNED(sum_out, 16)));
    hipStream_t st = (hipStream_t)stream;
    if (res)
        hipLaunchKernelGGL(rmsnorm_rows<true>, dim3(rows), dim3(kNormThreads), 0, st, (const uint16_t*)x,
                           (const uint16_t*)res, (const uint16_t*)w, (uint16_t*)sum_out, (uint16_t*)y, n, eps);
    else
        hipLaunchKernelGGL(rmsnorm_rows<false>, dim3(rows), dim3(kNormThreads), 0, st, (const uint16_t*)x,
                           (const uint16_t*)nullptr, (const uint16_t*)w, (uint16_t*)nullptr, (uint16_t*)y, n, eps);
    return moss_launch_status();
}

MOSS_API int moss_rmsnorm_quant_g32(const void* x, const void* res, const void* w, void* sum_out, void* y, void* qx,
                                    void* sx, void* qsum, int rows, int n, float eps, void* stream) {
    MOSS_CHECK_ARG(x && w && qx && sx && qsum && rows > 0 && n > 0 && n % 32 == 0 &&
                   n <= 8 * kNormThreads * kMaxChunks);
    MOSS_CHECK_ARG(MOSS_ALIGNED(x, 16) && MOSS_ALIGNED(w, 16) && MOSS_ALIGNED(y, 16) && MOSS_ALIGNED(qx, 8) &&
                   MOSS_ALIGNED(sx, 4) && MOSS_ALIGNED(qsum, 4));
    MOSS_CHECK_ARG(!res || (sum_out && MOSS_ALIGNED(res, 16) && MOSS_ALIGNED(sum_out, 16)));
    hipStream_t st = (hipStream_t)stream;
    if (res)
        hipLaunchKernelGGL((rmsnorm_rows<true, true>), dim3(rows), dim3(kNormThreads), 0, st, (const uint16_t*)x,
                           (const uint16_t*)res, (const uint16_t*)w, (uint16_t*)sum_out, (uint16_t*)y, n, eps,
                           (uint2*)qx, (float*)sx, (int*)qsum);
    else
        hipLaunchKernelGGL((rmsnorm_rows<false, true>), dim3(rows), dim3(kNormThreads), 0, st, (const uint16_t*)x,
                           (const uint16_t*)nullptr, (const uint16_t*)w, (uint16_t*)nullptr, (uint16_t*)y, n, eps,
                           (uint2*)qx, (float*)sx, (int*)qsum);
    return moss_launch_status();
}

MOSS_API int moss_qk_norm_rope_kv(const void* qkv, const void* q_weight, const void* k_weight, const void* cos,
                                  const void* sin, void* q_out, void* k_cache, void* v_cache, const void* positions,
                                  int L, int ntok, float eps, int cos_by_position, void* stream) {
    MOSS_CHECK_ARG(qkv && q_weight && k_weight && cos && sin && q_out && k_cache && v_cache && positions);
    MOSS_CHECK_ARG(L > 0 && ntok > 0);
    const int waves = ntok * 40;
    if (MOSS_ALIGNED(qkv, 8) && MOSS_ALIGNED(q_weight, 8) && MOSS_ALIGNED(k_weight, 8) && MOSS_ALIGNED(cos, 8) &&
        MOSS_ALIGNED(sin, 8) && MOSS_ALIGNED(q_out, 8) && MOSS_ALIGNED(k_cache, 8) && MOSS_ALIGNED(v_cache, 8)) {
        hipLaunchKernelGGL(qk_norm_rope_kv4<false>, dim3((waves + 15) / 16), dim3(256), 0, (hipStream_t)stream,
                           (const uint16_t*)qkv, (const uint16_t*)q_weight, (const uint16_t*)k_weight,
                           (const uint16_t*)cos, (const uint16_t*)sin, (uint16_t*)q_out, (uint16_t*)k_cache,
                           (uint16_t*)v_cache, (const int64_t*)positions, L, ntok, eps, cos_by_position);
        return moss_launch_status();
    }
    hipLaunchKernelGGL(qk_norm_rope_kv, dim3((waves + 3) / 4), dim3(256), 0, (hipStream_t)stream,
                       (const uint16_t*)qkv, (const uint16_t*)q_weight, (const uint16_t*)k_weight,
                       (const uint16_t*)cos, (const uint16_t*)sin, (uint16_t*)q_out, (uint16_t*)k_cache,
                       (uint16_t*)v_cache, (const int64_t*)positions, L, ntok, eps, cos_by_position);
    return moss_launch_status();
}

MOSS_API int moss_silu_mul(const void* x, void* y, int rows, int n, void* stream) {
    MOSS_CHECK_ARG(x && y && rows > 0 && n > 0 && n % 2 == 0 && MOSS_ALIGNED(x, 4) && MOSS_ALIGNED(y, 4));
    const size_t pairs = (size_t)rows * (n / 2);
    hipLaunchKernelGGL(silu_mul_rows, dim3((unsigned)((pairs + 255) / 256)), dim3(256), 0, (hipStream_t)stream,
                       (const uint32_t*)x, (uint32_t*)y, n, pairs);
    return moss_launch_status();
}
