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
// Combine order, the same in every kernel here so that all forms of a projection agree bit for
// bit: the groups of a row fall into slices of 64 (slice j = groups 64 j .. 64 j + 63); each
// group's term f32(isum) * (s_w * s_x) is rounded to fp32 on its own, a slice is summed by
// wave_sum's fixed tree, and the slice sums are added in slice order.
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

constexpr int kMaxSlices = 8;  // K <= 16384: at most 8 slices of 64 groups

// The integer dot of one group: sum (q - z) * qx over its 32 codes, exact in int32.
__device__ __forceinline__ int group_isum(const uint4& w, const uint4& xa, const uint4& xb, uint32_t zbyte,
                                          uint32_t zsh, int xq, uint32_t mask) {
    const uint32_t words[4] = {w.x, w.y, w.z, w.w};
    const uint32_t xw[8] = {xa.x, xa.y, xa.z, xa.w, xb.x, xb.y, xb.z, xb.w};
    int isum = -(int)((zbyte >> zsh) & 15u) * xq;
#pragma unroll
    for (int c = 0; c < 4; ++c) {
        isum = dot4(words[c] & mask, xw[2 * c], isum);
        isum = dot4((words[c] >> 4) & mask, xw[2 * c + 1], isum);
    }
    return isum;
}

// One slice's sum: the lane's group term rounded on its own (kept opaque, so the compiler cannot
// fuse it into the first add of the tree), then wave_sum's fixed tree.  A lane past the last
// group (live false) adds +0, as a zero weight does.
__device__ __forceinline__ float slice_sum(int isum, uint32_t s_bits, float xs, bool live = true) {
    float t = (float)isum * (bf16_bits((uint16_t)s_bits) * xs);
    t = live ? t : 0.f;
    asm volatile("" : "+v"(t));
    return wave_sum(t);
}

// Quantize one group of 32 bf16 values held as four 16-byte words, exactly as
// int8_quantize_g32 does: codes in dot4 order, the group scale and code sum.
__device__ __forceinline__ void quantize_group32(const uint4 (&h)[4], uint4& qa, uint4& qb, float& scale, int& sum) {
    float v[32];
#pragma unroll
    for (int c = 0; c < 4; ++c) {
        const uint32_t w[4] = {h[c].x, h[c].y, h[c].z, h[c].w};
#pragma unroll
        for (int p = 0; p < 4; ++p) {
            v[8 * c + 2 * p] = bf16_lo(w[p]);
            v[8 * c + 2 * p + 1] = bf16_hi(w[p]);
        }
    }
    float m = 0.f;
#pragma unroll
    for (int i = 0; i < 32; ++i) m = fmaxf(m, fabsf(v[i]));
    scale = g32_scale(m);
    const float inv = 1.0f / scale;
    uint32_t q[8];
    sum = 0;
#pragma unroll
    for (int c = 0; c < 4; ++c) sum += quantize8_dot4(v + 8 * c, inv, q[2 * c], q[2 * c + 1]);
    qa = make_uint4(q[0], q[1], q[2], q[3]);
    qb = make_uint4(q[4], q[5], q[6], q[7]);
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
// workgroup recomputes y = bf16(bf16(s * rsqrt(mean(s^2) + eps)) * w) of the one K-wide row
// (s = x, or bf16(x + res), which workgroup 0 also stores) and its int8 groups of 32 into LDS
// with its first 256 threads, while its weight rows are in flight.  Thread t owns the 8-value
// chunks t + 256 c (c < KG = K / 2048) and the 4 chunks of a group sit in one DPP quad, with the
// summation order and rounding points of rmsnorm_rows<RESIDUAL, true>, so the activations are
// bit-identical to moss_rmsnorm_quant_g32's.
struct W8Norm {
    const uint16_t* __restrict__ x;
    const uint16_t* __restrict__ res;
    const uint16_t* __restrict__ w;
    uint16_t* __restrict__ sum_out;
    float eps;
};

template <int KG>
struct W8NormLoad {
    uint4 x[KG], r[KG], w[KG];
};

// Issued before the weight loads (completions are counted in order); threads >= 256 load nothing.
template <int KG, int ACT>
__device__ __forceinline__ void w8norm_load(W8NormLoad<KG>& nl, const W8Norm& nm) {
    const int t = threadIdx.x;
    if (t >= 256) return;  // wave-uniform
#pragma unroll
    for (int c = 0; c < KG; ++c) {
        const int ci = t + 256 * c;
        nl.w[c] = reinterpret_cast<const uint4*>(nm.w)[ci];
        nl.x[c] = reinterpret_cast<const uint4*>(nm.x)[ci];
        if constexpr (ACT == 2) nl.r[c] = reinterpret_cast<const uint4*>(nm.res)[ci];
    }
}

// The normalized row quantized into LDS: lq[2 g .. 2 g + 1] (16 bytes) the codes of group g in
// dot4 order, lsx[g] its scale, lsum[g] its code sum.  Every thread of the workgroup calls it
// (two barriers).
template <int KG, int ACT>
__device__ __forceinline__ void w8norm_into_lds(const W8NormLoad<KG>& nl, const W8Norm& nm, uint2* lq, float* lsx,
                                                int* lsum, float* red, int G) {
    const int t = threadIdx.x, lane = t & (kWave - 1);
    const bool active = t < 256;  // wave-uniform
    float v[KG][8];
    float ss = 0.f;
#pragma unroll
    for (int c = 0; c < KG; ++c) {
        if (!active) break;
        const int ci = t + 256 * c;
        uint32_t sw[4] = {nl.x[c].x, nl.x[c].y, nl.x[c].z, nl.x[c].w};
        if constexpr (ACT == 2) {
            const uint32_t bw[4] = {nl.r[c].x, nl.r[c].y, nl.r[c].z, nl.r[c].w};
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
    if (lane == 0 && active) red[t / kWave] = ss;
    __syncthreads();
    float total = 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i) total += red[i];
    const float inv = rsqrtf(total / (float)(32 * G) + nm.eps);
#pragma unroll
    for (int c = 0; c < KG; ++c) {
        if (!active) break;
        const int ci = t + 256 * c;
        const uint32_t wv[4] = {nl.w[c].x, nl.w[c].y, nl.w[c].z, nl.w[c].w};
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
}

// The fused (add+)RMSNorm + quantizer + projection with K split: 8 waves per workgroup, KG
// slices of 64 groups (K = 2048 KG) times 8 / KG row groups of R rows (PAIRED: R gate and the R
// matching up rows); wave (slice, row group) takes the slice's groups of its rows, one per lane,
// and reads only its own group of the quantized row from LDS.  The slice sums meet in LDS and are
// added in slice order.  Against one wave per row holding the whole K (the same 8 rows per
// workgroup) the q||k||v projection goes from 6.0-6.3 to 5.3 us; the paired gate||up form takes
// 12 us against 13.6 us for the standalone norm + quantizer and the K-split gate||up.
template <int KG, int R, bool PAIRED, int ACT>
__global__ __launch_bounds__(512) void w4a8_ksplit_norm_kernel(const uint4* __restrict__ qw, const uint16_t* __restrict__ sc,
                                                               const uint8_t* __restrict__ zp, uint16_t* __restrict__ y,
                                                               int G, int n_out, W8Norm nm) {
    static_assert(KG == 1 || KG == 2 || KG == 4, "K = 2048, 4096 or 8192");
    constexpr int S = KG, RG = 8 / KG, NR = PAIRED ? 2 * R : R;
    const int t = threadIdx.x, lane = t & (kWave - 1);
    const int w = __builtin_amdgcn_readfirstlane(t / kWave);
    const int slice = w % S, rg = w / S;
    const int g = kWave * slice + lane;  // G = 64 KG: every lane's group exists
    const int rbase = blockIdx.x * RG * R, row0 = rbase + rg * R;
    W8NormLoad<KG> nl;
    w8norm_load<KG, ACT>(nl, nm);
    uint4 wv[NR];
    uint32_t s[NR], z[NR], zsh[NR];
#pragma unroll
    for (int r = 0; r < NR; ++r) {
        const int local = PAIRED ? (r % R) : r;
        const size_t n = (size_t)(min(row0 + local, n_out - 1) + ((PAIRED && r >= R) ? n_out : 0));
        const u32x4_t v = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(qw + n * G + g));
        wv[r] = make_uint4(v.x, v.y, v.z, v.w);
        s[r] = sc[n * G + g];
        int zb;
        zero_loc(g, G, zb, zsh[r]);
        z[r] = zp[n * (G >> 1) + zb];
    }
    __shared__ uint2 lq[256 * KG];
    __shared__ float lsx[64 * KG];
    __shared__ int lsum[64 * KG];
    __shared__ float red[4];
    __shared__ float part[S][RG * NR];
    w8norm_into_lds<KG, ACT>(nl, nm, lq, lsx, lsum, red, G);
    const uint4* p4 = reinterpret_cast<const uint4*>(lq) + 2 * g;
    const uint4 xa = p4[0], xb = p4[1];
    const float xs = lsx[g];
    const int xq = lsum[g];
    uint32_t mask = 0x0F0F0F0Fu;
    asm volatile("" : "+v"(mask));
#pragma unroll
    for (int r = 0; r < NR; ++r) {
        const float v = slice_sum(group_isum(wv[r], xa, xb, z[r], zsh[r], xq, mask), s[r], xs);
        if (lane == 0) part[slice][rg * NR + r] = v;
    }
    __syncthreads();
    if (t < RG * R && rbase + t < n_out) {
        const int pr = (t / R) * NR + t % R;  // row group t / R, local row t % R
        float a = part[0][pr], b = PAIRED ? part[0][pr + R] : 0.f;
#pragma unroll
        for (int i = 1; i < S; ++i) {
            a += part[i][pr];
            if constexpr (PAIRED) b += part[i][pr + R];
        }
        y[rbase + t] = PAIRED ? silu_mul_rounded_bits(a, b) : f32_to_bf16(a);
    }
}

// The paired gate||up GEMV with its output quantized for the next projection, row per wave:
// lane l owns groups l + 64 j (KG = ceil(G / 64)); 32 / R waves x R rows per workgroup cover
// one 32-row output group, which the workgroup also quantizes, as the reference's fused gate/up
// does (src/moss_tts/_runtime/dp4a_scaled.py:70-78).
template <int KG, int R>
__global__ __launch_bounds__(kWave * 32 / R) void w4a8_gemv_kernel(
    const uint32_t* __restrict__ qx, const float* __restrict__ sx, const int* __restrict__ qsum,
    const uint4* __restrict__ qw, const uint16_t* __restrict__ sc, const uint8_t* __restrict__ zp,
    uint16_t* __restrict__ y, uint8_t* __restrict__ oq, float* __restrict__ osx, int* __restrict__ osum, int G,
    int n_out) {
    static_assert(R == 2 || R == 4, "output quantization covers 32 paired rows");
    const int lane = threadIdx.x & (kWave - 1);
    const int wave = __builtin_amdgcn_readfirstlane(blockIdx.x * (blockDim.x / kWave) + (threadIdx.x / kWave));
    const int row0 = wave * R;
    // the grid holds whole 32-row groups (N_half % 32 == 0): no wave leaves early
    constexpr int NR = 2 * R;
    // activations first (completions are counted in order): 32 int8 per group, its scale and sum
    uint4 xa[KG], xb[KG];
    float xs[KG];
    int xq[KG];
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
    uint4 w[NR][KG];
    uint32_t s[NR][KG], z[NR][KG], zsh[NR][KG];  // z: the raw byte holding the zero point at bit zsh
#pragma unroll
    for (int r = 0; r < NR; ++r) {
        const int local = r % R;
        const int n = min(row0 + local, n_out - 1) + (r >= R ? n_out : 0);
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
    uint32_t mask = 0x0F0F0F0Fu;
    asm volatile("" : "+v"(mask));
    float out[NR];
#pragma unroll
    for (int r = 0; r < NR; ++r) {
        float acc = 0.f;
#pragma unroll
        for (int j = 0; j < KG; ++j) {  // lane l's group j lies in slice j
            const float t = slice_sum(group_isum(w[r][j], xa[j], xb[j], z[r][j], zsh[r][j], xq[j], mask), s[r][j], xs[j]);
            acc = j == 0 ? t : acc + t;
        }
        out[r] = acc;
    }
    uint16_t val[R];
#pragma unroll
    for (int r = 0; r < R; ++r) val[r] = silu_mul_rounded_bits(out[r], out[R + r]);
    if (lane == 0) {
#pragma unroll
        for (int r = 0; r < R; ++r)
            if (row0 + r < n_out) y[row0 + r] = val[r];
    }
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

// K-split GEMV: a workgroup of S = ceil(G / 64) waves owns R output rows (PAIRED: R gate and
// the R matching up rows); wave w takes slice w of every row, lane l the group 64 w + l, so a
// row's slices are read by S waves at once and the slice sums meet in LDS.  Against one wave per
// row holding all KG groups per lane this keeps S times as many waves in flight on the same
// bytes (K=12288, N=4096: 6.5 against 7.5 us).  QIN: the activations arrive as bf16 and each
// lane quantizes its own group in registers while the weight loads are in flight, bit-identical
// to int8_quantize_g32 and without its launch.
template <int R, bool PAIRED, bool QIN>
__global__ __launch_bounds__(kMaxSlices * kWave) void w4a8_ksplit_kernel(
    const uint32_t* __restrict__ qx, const float* __restrict__ sx, const int* __restrict__ qsum,
    const uint16_t* __restrict__ xb16, const uint4* __restrict__ qw, const uint16_t* __restrict__ sc,
    const uint8_t* __restrict__ zp, uint16_t* __restrict__ y, int G, int n_out) {
    constexpr int NR = PAIRED ? 2 * R : R;
    const int lane = threadIdx.x & (kWave - 1);
    const int slice = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
    const int g = kWave * slice + lane;
    // The last slice may be partial: its dead lanes load group G - 1 (in bounds, no branch around
    // the loads) and add +0 in slice_sum.
    const bool live = g < G;
    const int gc = min(g, G - 1);
    const int row0 = blockIdx.x * R;
    // activations first (completions are counted in order)
    uint4 xa, xb, h[4];
    float xs;
    int xq;
    if constexpr (QIN) {
#pragma unroll
        for (int c = 0; c < 4; ++c) h[c] = reinterpret_cast<const uint4*>(xb16 + 32 * gc)[c];
    } else {
        const uint4* p = reinterpret_cast<const uint4*>(qx + 8 * gc);
        xa = p[0];
        xb = p[1];
        xs = sx[gc];
        xq = qsum[gc];
    }
    uint4 w[NR];
    uint32_t s[NR], z[NR], zsh[NR];
#pragma unroll
    for (int r = 0; r < NR; ++r) {
        const int local = PAIRED ? (r % R) : r;
        const size_t n = (size_t)(min(row0 + local, n_out - 1) + ((PAIRED && r >= R) ? n_out : 0));
        const u32x4_t v = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(qw + n * G + gc));
        w[r] = make_uint4(v.x, v.y, v.z, v.w);
        s[r] = sc[n * G + gc];
        int zb;
        zero_loc(gc, G, zb, zsh[r]);
        z[r] = zp[n * (G >> 1) + zb];
    }
    if constexpr (QIN) {
        // every weight load is issued before the quantization waits for the activations
        __builtin_amdgcn_sched_barrier(0);
        quantize_group32(h, xa, xb, xs, xq);
    }
    uint32_t mask = 0x0F0F0F0Fu;
    asm volatile("" : "+v"(mask));
    __shared__ float part[kMaxSlices][NR];
#pragma unroll
    for (int r = 0; r < NR; ++r) {
        const float t = slice_sum(group_isum(w[r], xa, xb, z[r], zsh[r], xq, mask), s[r], xs, live);
        if (lane == 0) part[slice][r] = t;
    }
    __syncthreads();
    const int t = threadIdx.x, S = blockDim.x / kWave;
    if (t < R && row0 + t < n_out) {
        float a = part[0][t], b = PAIRED ? part[0][R + t] : 0.f;
        for (int i = 1; i < S; ++i) {
            a += part[i][t];
            if (PAIRED) b += part[i][R + t];
        }
        y[row0 + t] = PAIRED ? silu_mul_rounded_bits(a, b) : f32_to_bf16(a);
    }
}

template <bool PAIRED, bool QIN>
int launch_w4a8_ksplit(const void* qx, const void* sx, const void* qsum, const void* xb16, const void* qw,
                       const void* sc, const void* zp, void* y, int K, int n_out, int rows, hipStream_t st) {
    const int G = K / 32, S = (G + kWave - 1) / kWave;
    if (S > kMaxSlices) return (int)hipErrorInvalidValue;
    // measured: 4 rows for the 6-slice K=12288 down projection, 2 for K=4096 (O, q||k||v, gate||up)
    const int R = rows ? rows : (!PAIRED && S >= 4 ? 4 : 2);
    const dim3 grid((n_out + R - 1) / R), block(kWave * S);
#define MOSS_W4A8K(RV)                                                                                            \
    if (R == RV) {                                                                                                \
        hipLaunchKernelGGL((w4a8_ksplit_kernel<RV, PAIRED, QIN>), grid, block, 0, st, (const uint32_t*)qx,         \
                           (const float*)sx, (const int*)qsum, (const uint16_t*)xb16, (const uint4*)qw,           \
                           (const uint16_t*)sc, (const uint8_t*)zp, (uint16_t*)y, G, n_out);                      \
        return moss_launch_status();                                                                              \
    }
    MOSS_W4A8K(1) MOSS_W4A8K(2) MOSS_W4A8K(4)
#undef MOSS_W4A8K
    return (int)hipErrorInvalidValue;
}

// The paired gate||up with its output quantized (32 output rows per workgroup).
int launch_w4a8_qout(const void* qx, const void* sx, const void* qsum, const void* qw, const void* sc, const void* zp,
                     void* y, void* oq, void* osx, void* osum, int K, int n_out, int rows, hipStream_t st) {
    const int G = K / 32, KG = (G + kWave - 1) / kWave;
    if (rows == 0) rows = 2;
    const int wpb = 32 / rows;
    const dim3 grid((n_out + 31) / 32), block(kWave * wpb);
#define MOSS_W4A8(KGV, RV)                                                                                        \
    if (KG == KGV && rows == RV) {                                                                                \
        hipLaunchKernelGGL((w4a8_gemv_kernel<KGV, RV>), grid, block, 0, st, (const uint32_t*)qx, (const float*)sx, \
                           (const int*)qsum, (const uint4*)qw, (const uint16_t*)sc, (const uint8_t*)zp,           \
                           (uint16_t*)y, (uint8_t*)oq, (float*)osx, (int*)osum, G, n_out);                        \
        return moss_launch_status();                                                                              \
    }
#define MOSS_W4A8_R(KGV) MOSS_W4A8(KGV, 2) MOSS_W4A8(KGV, 4)
    MOSS_W4A8_R(1) MOSS_W4A8_R(2) MOSS_W4A8_R(3) MOSS_W4A8_R(4) MOSS_W4A8_R(5) MOSS_W4A8_R(6) MOSS_W4A8_R(7)
    MOSS_W4A8_R(8)
#undef MOSS_W4A8_R
#undef MOSS_W4A8
    return (int)hipErrorInvalidValue;
}

// K = 2048 KG, KG in {1, 2, 4} (K = 2048, 4096, 8192); rows per wave 1, 2 or 4 (0: 2, measured
// best for the q||k||v projection).
template <bool PAIRED>
int launch_w4a8_norm(const W8Norm& nm, const void* qw, const void* sc, const void* zp, void* y, int K, int n_out,
                     int rows, hipStream_t st) {
    const int G = K / 32, KG = K / 2048;
    if (rows == 0) rows = 2;
    const int per_block = (8 / KG) * rows;
    const dim3 grid((n_out + per_block - 1) / per_block), block(512);
#define MOSS_W4A8N(KGV, RV, ACTV)                                                                                 \
    if (KG == KGV && rows == RV) {                                                                                \
        hipLaunchKernelGGL((w4a8_ksplit_norm_kernel<KGV, RV, PAIRED, ACTV>), grid, block, 0, st, (const uint4*)qw, \
                           (const uint16_t*)sc, (const uint8_t*)zp, (uint16_t*)y, G, n_out, nm);                  \
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
    return launch_w4a8_ksplit<false, false>(qx, sx, qsum, nullptr, qw, sc, zp, y, K, N, rows_per_wave,
                                            (hipStream_t)stream);
}

MOSS_API int moss_w4a8_quant_gemv(const void* x, const void* qw, const void* sc, const void* zp, void* y, int K, int N,
                                  int rows_per_wave, void* stream) {
    MOSS_CHECK_ARG(x && qw && sc && zp && y && K > 0 && K % 64 == 0 && K <= 16384 && N > 0);
    MOSS_CHECK_ARG(rows_per_wave == 0 || rows_per_wave == 1 || rows_per_wave == 2 || rows_per_wave == 4);
    MOSS_CHECK_ARG(MOSS_ALIGNED(x, 16) && MOSS_ALIGNED(qw, 16));
    return launch_w4a8_ksplit<false, true>(nullptr, nullptr, nullptr, x, qw, sc, zp, y, K, N, rows_per_wave,
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
        return launch_w4a8_ksplit<true, false>(qx, sx, qsum, nullptr, qw, sc, zp, y, K, N_half, rows_per_wave,
                                               (hipStream_t)stream);
    MOSS_CHECK_ARG(N_half % 32 == 0 && rows_per_wave != 1);
    MOSS_CHECK_ARG(MOSS_ALIGNED(out_sx, 4) && MOSS_ALIGNED(out_qsum, 4));
    return launch_w4a8_qout(qx, sx, qsum, qw, sc, zp, y, out_qx, out_sx, out_qsum, K, N_half, rows_per_wave,
                            (hipStream_t)stream);
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
