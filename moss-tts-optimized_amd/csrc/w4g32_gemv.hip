// Batch-1 INT4 group-32 GEMV (W4A16) and the fused gate||up SiLU*mul variant.
//
// y[n] = sum_g s[n,g] * sum_{k in g} (q[n,k] - z[n,g]) * x[k]     (fp32 accumulate, bf16 out)
//
// Mapping (gfx950, wave64): one wave owns R output rows; its 64 lanes split K, lane l
// owning groups l, l+64, l+128, ... (16 bytes of codes per group, so each global_load_dwordx4
// of a wave reads 1 KiB contiguous).  The lane's slice of x stays in VGPRs for all R rows.
// Unrounded mode: codes become bf16 lanes with one and-or: (w >> 4i) & 0x000F000F | 0x43004300
// is the pair (128 + q_2i, 128 + q_2i+1), exact in bf16, fed to v_dot2_f32_bf16 against the
// matching x pair; per group sum (q - z) x = acc - (128 + z) * sum_g x, then * s.  Exact mode:
// every weight is dequantized bit-exactly first (dequant_word_mixed), then meets its x pair in
// v_dot2_f32_bf16.  Rows are reduced with DPP (no LDS, no atomics, no workspace): every output
// element is written once.
//
// Reference semantics: dequant-then-matmul of src/moss_tts/calibration.py:185-188 with
// src/moss_tts/_runtime/calibrated_quant.py:41-42; paired epilogue rounding points of
// src/moss_tts/_runtime/dp4a_scaled.py:65-68 (gate, up, SiLU and product rounded to bf16).
#include "common.h"
#include "norm_fused.h"

namespace moss {
namespace {

template <int KG>
struct XSlice {
    uint32_t v[KG][16];  // 32 bf16 of group (lane + 64 j), as 16 packed pairs
    float sum[KG];       // fp32 sum of those 32 values
};

template <int KG, bool SUMS, bool FULL>
__device__ __forceinline__ void load_x(XSlice<KG>& xs, const uint16_t* __restrict__ x, int lane, int G) {
    uint32_t ones = 0x3F803F80u;  // bf16 pair (1.0, 1.0): group sums through the same dot2 path
    asm volatile("" : "+v"(ones));
#pragma unroll
    for (int j = 0; j < KG; ++j) {
        const int g = lane + kWave * j;
        float s = 0.f;
        if (FULL || g < G) {
            const uint4* p = reinterpret_cast<const uint4*>(x + 32 * g);
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                const uint4 t = p[c];
                xs.v[j][4 * c + 0] = t.x;
                xs.v[j][4 * c + 1] = t.y;
                xs.v[j][4 * c + 2] = t.z;
                xs.v[j][4 * c + 3] = t.w;
            }
            if constexpr (SUMS) {
#pragma unroll
                for (int m = 0; m < 16; ++m) s = dot2_bf16(xs.v[j][m], ones, s);
            }
        } else {
#pragma unroll
            for (int m = 0; m < 16; ++m) xs.v[j][m] = 0u;
        }
        xs.sum[j] = s;
    }
}

template <int KG>
struct RowLoad {
    uint4 w[KG];
    uint32_t s[KG];  // bf16 scale bits
    uint32_t z[KG];  // zero point
};

// FULL: G == 64 * KG with KG even: every 128-group block is complete, so byte 64 jj + l of
// the zp row holds lane l's zeros for groups l + 128 jj (low) and l + 128 jj + 64 (high).
template <int KG, bool FULL>
__device__ __forceinline__ void load_row(RowLoad<KG>& r, const uint4* __restrict__ qw,
                                         const uint16_t* __restrict__ sc, const uint8_t* __restrict__ zp,
                                         int n, int lane, int G) {
    const int h = G >> 1;
    if constexpr (FULL) {
#pragma unroll
        for (int j = 0; j < KG; ++j) {
            r.w[j] = qw[(size_t)n * G + lane + kWave * j];
            r.s[j] = sc[(size_t)n * G + lane + kWave * j];
        }
#pragma unroll
        for (int jj = 0; jj < KG / 2; ++jj) {
            const uint32_t b = zp[(size_t)n * h + lane + kWave * jj];
            r.z[2 * jj] = b & 15u;
            r.z[2 * jj + 1] = b >> 4;
        }
    } else {
#pragma unroll
        for (int j = 0; j < KG; ++j) {
            const int g = lane + kWave * j;
            if (g < G) {
                r.w[j] = qw[(size_t)n * G + g];
                r.s[j] = sc[(size_t)n * G + g];
                r.z[j] = zero_of_group(zp + (size_t)n * h, g, G);
            } else {
                r.w[j] = make_uint4(0u, 0u, 0u, 0u);
                r.s[j] = 0u;
                r.z[j] = 0u;
            }
        }
    }
}

// Constants pinned in VGPRs so each code pair costs one v_and_or_b32 (a VOP3 form, which
// on gfx9 takes no literal operand) after its shift.
struct Magic {
    uint32_t mask, bias;
};

__device__ __forceinline__ Magic make_magic() {
    Magic m{0x000F000Fu, 0x43004300u};
    asm volatile("" : "+v"(m.mask), "+v"(m.bias));
    return m;
}

__device__ __forceinline__ float word_dot(uint32_t w, const uint32_t* xv, float acc, Magic m) {
#pragma unroll
    for (int i = 0; i < 4; ++i) acc = dot2_bf16(((w >> (4 * i)) & m.mask) | m.bias, xv[i], acc);
    return acc;
}

// Unrounded form: sum_g s * (sum (128+q) x - (128+z) sum x); weights are never rounded.
template <int KG>
__device__ __forceinline__ float row_partial_unrounded(const XSlice<KG>& xs, const RowLoad<KG>& r, Magic m) {
    float part = 0.f;
#pragma unroll
    for (int j = 0; j < KG; ++j) {
        // the chain starts at -(128 + z) * sum(x): it ends at sum (q - z) x directly
        float acc = -(128.0f + (float)r.z[j]) * xs.sum[j];
        acc = word_dot(r.w[j].x, &xs.v[j][0], acc, m);
        acc = word_dot(r.w[j].y, &xs.v[j][4], acc, m);
        acc = word_dot(r.w[j].z, &xs.v[j][8], acc, m);
        acc = word_dot(r.w[j].w, &xs.v[j][12], acc, m);
        part = fmaf(bf16_bits((uint16_t)r.s[j]), acc, part);
    }
    return part;
}

// Exact form: every weight is the bit-exact bf16 dequant bf16_rne((q - z) * s) before it
// meets x (dequant_word_mixed, four pairs at a time), then a dot2 with the matching x pair
// accumulates in fp32.
__device__ __forceinline__ float word_dot_exact(uint32_t w, const uint32_t* xv, float acc, const MixedUnpack& c,
                                                const GroupDequant& gd) {
    uint32_t wq[4];
    dequant_word_mixed(w, c, gd.s_lo, gd.s_hi, gd.s, gd.bias_bf16, gd.bias_f16, wq);
#pragma unroll
    for (int i = 0; i < 4; ++i) acc = dot2_bf16(wq[i], xv[i], acc);
    return acc;
}

template <int KG>
__device__ __forceinline__ float row_partial_exact(const XSlice<KG>& xs, const RowLoad<KG>& r, const MixedUnpack& c) {
    float acc = 0.f;  // one dot2 chain over the whole row: the weights already carry their scale
#pragma unroll
    for (int j = 0; j < KG; ++j) {
        const GroupDequant gd = group_dequant(r.s[j], r.z[j]);
        acc = word_dot_exact(r.w[j].x, &xs.v[j][0], acc, c, gd);
        acc = word_dot_exact(r.w[j].y, &xs.v[j][4], acc, c, gd);
        acc = word_dot_exact(r.w[j].z, &xs.v[j][8], acc, c, gd);
        acc = word_dot_exact(r.w[j].w, &xs.v[j][12], acc, c, gd);
    }
    return acc;
}

// The exact form over the normalized row in LDS (the fused-norm kernels), group by group: the
// lane's x group j (16 packed pairs) is read once for all rows, then group j + 1, so one group of
// x is held at a time (16 VGPRs instead of 16 KG: the gate||up kernel fits 5 waves per SIMD
// instead of 4).  Every row's chain visits its words in row_partial_exact's order, so the sums
// are bit-identical to it.  NORM > 0 means G = 64 KG: every group of every lane exists.
template <int KG, int NR>
__device__ __forceinline__ void rows_exact_from_lds(const uint16_t* xn, const RowLoad<KG> (&rows)[NR], int lane,
                                                    float (&acc)[NR]) {
    const MixedUnpack c = make_mixed_unpack();
#pragma unroll
    for (int r = 0; r < NR; ++r) acc[r] = 0.f;
#pragma unroll
    for (int j = 0; j < KG; ++j) {
        uint32_t xv[16];
        const uint4* p = reinterpret_cast<const uint4*>(xn + 32 * (lane + kWave * j));
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const uint4 v = p[q];
            xv[4 * q] = v.x;
            xv[4 * q + 1] = v.y;
            xv[4 * q + 2] = v.z;
            xv[4 * q + 3] = v.w;
        }
#pragma unroll
        for (int r = 0; r < NR; ++r) {
            const GroupDequant gd = group_dequant(rows[r].s[j], rows[r].z[j]);
            acc[r] = word_dot_exact(rows[r].w[j].x, &xv[0], acc[r], c, gd);
            acc[r] = word_dot_exact(rows[r].w[j].y, &xv[4], acc[r], c, gd);
            acc[r] = word_dot_exact(rows[r].w[j].z, &xv[8], acc[r], c, gd);
            acc[r] = word_dot_exact(rows[r].w[j].w, &xv[12], acc[r], c, gd);
        }
        __builtin_amdgcn_sched_barrier(0);  // the next group's LDS reads stay after these products
    }
}

typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));

// Non-temporal loads: every weight byte is read once.
template <int KG, bool FULL>
__device__ __forceinline__ void load_row_nt(RowLoad<KG>& r, const uint4* __restrict__ qw,
                                            const uint16_t* __restrict__ sc, const uint8_t* __restrict__ zp,
                                            int n, int lane, int G) {
    const int h = G >> 1;
#pragma unroll
    for (int j = 0; j < KG; ++j) {
        const int g = lane + kWave * j;
        if (FULL || g < G) {
            const u32x4_t v = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(qw + (size_t)n * G + g));
            r.w[j] = make_uint4(v.x, v.y, v.z, v.w);
            r.s[j] = __builtin_nontemporal_load(sc + (size_t)n * G + g);
        } else {
            r.w[j] = make_uint4(0u, 0u, 0u, 0u);
            r.s[j] = 0u;
        }
    }
    if constexpr (FULL) {
#pragma unroll
        for (int jj = 0; jj < KG / 2; ++jj) {
            const uint32_t b = __builtin_nontemporal_load(zp + (size_t)n * h + lane + kWave * jj);
            r.z[2 * jj] = b & 15u;
            r.z[2 * jj + 1] = b >> 4;
        }
    } else {
#pragma unroll
        for (int j = 0; j < KG; ++j) {
            const int g = lane + kWave * j;
            if (g < G) {
                r.z[j] = zero_of_group(zp + (size_t)n * h, g, G);
            } else {
                r.z[j] = 0u;
            }
        }
    }
}


// n_out output rows; PAIRED reads gate row n and up row n + n_out.  NORM > 0 needs
// K = 2048 KG (the whole workgroup takes part in the normalization, so no wave leaves early).
template <int KG, int R, bool PAIRED, bool FULL, bool EXACT, int NORM>
__device__ __forceinline__ void gemv_rows(const uint16_t* __restrict__ x, const uint4* __restrict__ qw,
                                          const uint16_t* __restrict__ sc, const uint8_t* __restrict__ zp,
                                          uint16_t* __restrict__ y, int G, int n_out, const NormArgs& na) {
    const int lane = threadIdx.x & (kWave - 1);
    // wave-uniform: lets row addressing run on the scalar unit
    const int wave = __builtin_amdgcn_readfirstlane(blockIdx.x * (blockDim.x / kWave) + (threadIdx.x / kWave));
    const int row0 = wave * R;
    if (NORM == 0 && row0 >= n_out) return;  // wave-uniform

    constexpr int NR = PAIRED ? 2 * R : R;
    // The activations are loaded before the weight rows: vector-memory completions are counted
    // in order, so row 0 can then be computed while later rows are still arriving.
    NormLoad<(NORM > 0 ? KG : 1)> nl;
    XSlice<KG> xs;
    if constexpr (NORM > 0) norm_load<NORM, KG>(nl, x, na);
    else load_x<KG, !EXACT, FULL>(xs, x, lane, G);
    RowLoad<KG> rows[NR];
#pragma unroll
    for (int r = 0; r < NR; ++r) {
        const int local = PAIRED ? (r % R) : r;
        const int n = min(row0 + local, n_out - 1) + ((PAIRED && r >= R) ? n_out : 0);
        load_row_nt<KG, FULL>(rows[r], qw, sc, zp, n, lane, G);
    }
    float out[NR];
    if constexpr (NORM > 0) {
        __shared__ __attribute__((aligned(16))) uint16_t xn[2048 * KG];
        __shared__ float red[4];
        norm_into_lds<NORM, KG>(nl, na, xn, red, 32 * G);
        if (row0 >= n_out) return;  // after the workgroup's barriers
        if constexpr (EXACT) {
            rows_exact_from_lds<KG, NR>(xn, rows, lane, out);
        } else {
            load_x<KG, true, FULL>(xs, xn, lane, G);
            const Magic m = make_magic();
#pragma unroll
            for (int r = 0; r < NR; ++r) out[r] = row_partial_unrounded(xs, rows[r], m);
        }
    } else if constexpr (EXACT) {
        const MixedUnpack c = make_mixed_unpack();
#pragma unroll
        for (int r = 0; r < NR; ++r) out[r] = row_partial_exact(xs, rows[r], c);
    } else {
        const Magic m = make_magic();
#pragma unroll
        for (int r = 0; r < NR; ++r) out[r] = row_partial_unrounded(xs, rows[r], m);
    }
#pragma unroll
    for (int r = 0; r < NR; ++r) out[r] = wave_sum(out[r]);

    if (lane == 0) {
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const int n = row0 + r;
            if (n < n_out) y[n] = PAIRED ? silu_mul_rounded_bits(out[r], out[R + r]) : f32_to_bf16(out[r]);
        }
    }
}

// ---------------------------------------------------------------------------------------
// Large K (K = 4096 W): the W waves of a workgroup each own one 4096-wide slice of K (128
// groups, lane l holding groups 128 s + l and 128 s + l + 64), so every wave keeps the
// 32-VGPR x slice of the K = 4096 case; the per-slice row sums meet in LDS and are added in
// slice order by wave 0.
template <bool NT>
__device__ __forceinline__ void load_row_slice(RowLoad<2>& r, const uint4* __restrict__ qw,
                                               const uint16_t* __restrict__ sc, const uint8_t* __restrict__ zp,
                                               int n, int lane, int G, int g0) {
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        const size_t gi = (size_t)n * G + g0 + lane + kWave * j;
        if constexpr (NT) {
            const u32x4_t v = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(qw + gi));
            r.w[j] = make_uint4(v.x, v.y, v.z, v.w);
            r.s[j] = __builtin_nontemporal_load(sc + gi);
        } else {
            r.w[j] = qw[gi];
            r.s[j] = sc[gi];
        }
    }
    // block g0 / 128 is complete: byte g0 / 2 + lane holds this lane's two zero points
    const size_t zi = (size_t)n * (G >> 1) + (g0 >> 1) + lane;
    const uint32_t b = NT ? (uint32_t)__builtin_nontemporal_load(zp + zi) : (uint32_t)zp[zi];
    r.z[0] = b & 15u;
    r.z[1] = b >> 4;
}

template <int W, int R, bool PAIRED, bool EXACT>
__device__ __forceinline__ void gemv_ksplit(const uint16_t* __restrict__ x, const uint4* __restrict__ qw,
                                            const uint16_t* __restrict__ sc, const uint8_t* __restrict__ zp,
                                            uint16_t* __restrict__ y, int G, int n_out) {
    constexpr int NR = PAIRED ? 2 * R : R;
    __shared__ float part[W][NR];
    const int lane = threadIdx.x & (kWave - 1);
    const int slice = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
    const int row0 = blockIdx.x * R;
    if (row0 >= n_out) return;  // uniform across the workgroup
    const int g0 = 128 * slice;

    XSlice<2> xs;
    load_x<2, !EXACT, true>(xs, x + 32 * g0, lane, 128);  // first: see gemv_rows
    RowLoad<2> rows[NR];
#pragma unroll
    for (int r = 0; r < NR; ++r) {
        const int local = PAIRED ? (r % R) : r;
        const int n = min(row0 + local, n_out - 1) + ((PAIRED && r >= R) ? n_out : 0);
        load_row_slice<true>(rows[r], qw, sc, zp, n, lane, G, g0);
    }
    float v[NR];
    if constexpr (EXACT) {
        const MixedUnpack c = make_mixed_unpack();
#pragma unroll
        for (int r = 0; r < NR; ++r) v[r] = wave_sum(row_partial_exact(xs, rows[r], c));
    } else {
        const Magic m = make_magic();
#pragma unroll
        for (int r = 0; r < NR; ++r) v[r] = wave_sum(row_partial_unrounded(xs, rows[r], m));
    }
    if (lane == 0) {
#pragma unroll
        for (int r = 0; r < NR; ++r) part[slice][r] = v[r];
    }
    __syncthreads();
    if (slice == 0 && lane < R) {
        const int n = row0 + lane;
        if (n < n_out) {
            float a = 0.f, b = 0.f;
#pragma unroll
            for (int w = 0; w < W; ++w) {
                a += part[w][lane];
                if constexpr (PAIRED) b += part[w][R + lane];
            }
            y[n] = PAIRED ? silu_mul_rounded_bits(a, b) : f32_to_bf16(a);
        }
    }
}

// ---------------------------------------------------------------------------------------
// A few tokens (M = 2 .. kMaxTokens, exact mode): R weight rows per wave, each dequantized once
// and multiplied with the x slice of every token (T slices held in VGPRs), so the weights are
// read once for all T rows of y, on the VALU (no matrix-core instruction).  Each token's dot is
// row_partial_exact's chain over the same words in the same order, followed by the same
// wave_sum: every row of y equals the single-token GEMV of that token bit for bit.
constexpr int kMaxTokens = 4;

template <int KG, int T>
__device__ __forceinline__ void row_partial_exact_tokens(const XSlice<KG> (&xs)[T], const RowLoad<KG>& r,
                                                         const MixedUnpack& c, float (&acc)[T]) {
#pragma unroll
    for (int t = 0; t < T; ++t) acc[t] = 0.f;
#pragma unroll
    for (int j = 0; j < KG; ++j) {
        const GroupDequant gd = group_dequant(r.s[j], r.z[j]);
        const uint32_t words[4] = {r.w[j].x, r.w[j].y, r.w[j].z, r.w[j].w};
#pragma unroll
        for (int wd = 0; wd < 4; ++wd) {
            uint32_t wq[4];
            dequant_word_mixed(words[wd], c, gd.s_lo, gd.s_hi, gd.s, gd.bias_bf16, gd.bias_f16, wq);
#pragma unroll
            for (int t = 0; t < T; ++t)
#pragma unroll
                for (int i = 0; i < 4; ++i) acc[t] = dot2_bf16(wq[i], xs[t].v[j][4 * wd + i], acc[t]);
        }
    }
}

// x bf16 [T, 32 G], y bf16 [T, n_out]; R weight rows per wave, grid ceil(n_out / (4 R))
// workgroups of 4 waves.
template <int KG, int T, int R, bool FULL>
__global__ __launch_bounds__(256) void w4g32_gemv_tokens_exact(const uint16_t* __restrict__ x,
                                                               const uint4* __restrict__ qw,
                                                               const uint16_t* __restrict__ sc,
                                                               const uint8_t* __restrict__ zp,
                                                               uint16_t* __restrict__ y, int G, int n_out) {
    const int lane = threadIdx.x & (kWave - 1);
    const int wave = __builtin_amdgcn_readfirstlane(blockIdx.x * (blockDim.x / kWave) + (threadIdx.x / kWave));
    const int row0 = wave * R;
    if (row0 >= n_out) return;  // wave-uniform
    XSlice<KG> xs[T];
#pragma unroll
    for (int t = 0; t < T; ++t) load_x<KG, false, FULL>(xs[t], x + (size_t)t * 32 * G, lane, G);
    RowLoad<KG> rows[R];
#pragma unroll
    for (int r = 0; r < R; ++r) load_row_nt<KG, FULL>(rows[r], qw, sc, zp, min(row0 + r, n_out - 1), lane, G);
    const MixedUnpack c = make_mixed_unpack();
#pragma unroll
    for (int r = 0; r < R; ++r) {
        float acc[T];
        row_partial_exact_tokens<KG, T>(xs, rows[r], c, acc);
#pragma unroll
        for (int t = 0; t < T; ++t) {
            const float v = wave_sum(acc[t]);
            if (lane == 0 && row0 + r < n_out) y[(size_t)t * n_out + row0 + r] = f32_to_bf16(v);
        }
    }
}

// Large K (K = 4096 W, as gemv_ksplit): workgroup = R weight rows, wave s = K slice s; the
// slices' sums meet in LDS and are added in slice order, as gemv_ksplit adds them.
template <int W, int T, int R>
__global__ __launch_bounds__(64 * W) void w4g32_gemv_ksplit_tokens_exact(const uint16_t* __restrict__ x,
                                                                        const uint4* __restrict__ qw,
                                                                        const uint16_t* __restrict__ sc,
                                                                        const uint8_t* __restrict__ zp,
                                                                        uint16_t* __restrict__ y, int G, int n_out) {
    __shared__ float part[W][R][T];
    const int lane = threadIdx.x & (kWave - 1);
    const int slice = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
    const int row0 = blockIdx.x * R;  // < n_out (grid)
    const int g0 = 128 * slice;
    XSlice<2> xs[T];
#pragma unroll
    for (int t = 0; t < T; ++t) load_x<2, false, true>(xs[t], x + (size_t)t * 32 * G + 32 * g0, lane, 128);
    RowLoad<2> rows[R];
#pragma unroll
    for (int r = 0; r < R; ++r) load_row_slice<true>(rows[r], qw, sc, zp, min(row0 + r, n_out - 1), lane, G, g0);
    const MixedUnpack c = make_mixed_unpack();
#pragma unroll
    for (int r = 0; r < R; ++r) {
        float acc[T];
        row_partial_exact_tokens<2, T>(xs, rows[r], c, acc);
#pragma unroll
        for (int t = 0; t < T; ++t) {
            const float v = wave_sum(acc[t]);
            if (lane == 0) part[slice][r][t] = v;
        }
    }
    __syncthreads();
    if (slice == 0 && lane < R * T) {
        const int r = lane / T, t = lane % T;
        if (row0 + r < n_out) {
            float a = 0.f;
#pragma unroll
            for (int w = 0; w < W; ++w) a += part[w][r][t];
            y[(size_t)t * n_out + row0 + r] = f32_to_bf16(a);
        }
    }
}

template <int T>
int launch_tokens_t(const void* x, const void* qw, const void* sc, const void* zp, void* y, int G, int n_out,
                    hipStream_t st) {
    const auto* xp = (const uint16_t*)x;
    const auto* qp = (const uint4*)qw;
    const auto* sp = (const uint16_t*)sc;
    const auto* zpp = (const uint8_t*)zp;
    auto* yp = (uint16_t*)y;
    // K = 4096 W for W = 2, 3, 4: the K-split form (as the single-token GEMV splits those K)
    if (G % 128 == 0 && G >= 256 && G <= 512) {
        // 4 rows per workgroup (measured on MI355X at K = 8192 and 12288, N = 4096, 2 to 4 tokens:
        // 1 row 11.3-28.0 us, 2 rows 8.1-17.3, 4 rows 7.5-15.2)
        const int W = G / 128;
        const dim3 grid((n_out + 3) / 4);
#define MOSS_TK(WV)                                                                                                 \
    if (W == WV) {                                                                                                  \
        hipLaunchKernelGGL((w4g32_gemv_ksplit_tokens_exact<WV, T, 4>), grid, dim3(64 * WV), 0, st, xp, qp, sp, zpp, \
                           yp, G, n_out);                                                                           \
        return moss_launch_status();                                                                                \
    }
        MOSS_TK(2) MOSS_TK(3) MOSS_TK(4)
#undef MOSS_TK
        return (int)hipErrorInvalidValue;
    }
    const int KG = (G + kWave - 1) / kWave;
    if (KG > 2) return (int)hipErrorInvalidValue;  // T x KG x 16 VGPRs of x: K <= 4096
    const bool full = (G == kWave * KG) && (KG % 2 == 0);
    // 4 rows per wave unless 2 fill the CUs in fewer row-rounds (a round: every CU holding one
    // workgroup of 4 waves).  Measured on MI355X, K = 4096, 2 to 4 tokens: N = 4096 / 12288 / 24576
    // fastest at 4 rows, N = 6144 at 2 (384 workgroups of 4 rows leave half a round).
    const int wg4 = (n_out + 15) / 16, wg2 = (n_out + 7) / 8;
    const int R = ((wg2 + 255) / 256) * 2 < ((wg4 + 255) / 256) * 4 ? 2 : 4;
    const dim3 block(256);
#define MOSS_TR(RV)                                                                                                 \
    if (R == RV) {                                                                                                  \
        const dim3 grid((n_out + 4 * RV - 1) / (4 * RV));                                                           \
        if (KG == 1)                                                                                                \
            hipLaunchKernelGGL((w4g32_gemv_tokens_exact<1, T, RV, false>), grid, block, 0, st, xp, qp, sp, zpp, yp, \
                               G, n_out);                                                                           \
        else if (full)                                                                                              \
            hipLaunchKernelGGL((w4g32_gemv_tokens_exact<2, T, RV, true>), grid, block, 0, st, xp, qp, sp, zpp, yp,  \
                               G, n_out);                                                                           \
        else                                                                                                        \
            hipLaunchKernelGGL((w4g32_gemv_tokens_exact<2, T, RV, false>), grid, block, 0, st, xp, qp, sp, zpp, yp, \
                               G, n_out);                                                                           \
        return moss_launch_status();                                                                                \
    }
    MOSS_TR(2) MOSS_TR(4)
#undef MOSS_TR
    return (int)hipErrorInvalidValue;
}

// ---------------------------------------------------------------------------------------
// Entry kernels: one name per (role, dequant mode), so profiles tell them apart.
// The plain GEMV at up to 2 rows per wave fits 6 waves per SIMD (80 VGPRs), so a K = 4096,
// N = 12288 launch (1536 workgroups) runs in one round on 256 CUs instead of 1.2.
#define MOSS_ROWS_WAVES(PAIRED, NORM, R) ((!(PAIRED) && (NORM) == 0 && (R) <= 2) ? 6 : 1)
#define MOSS_ROWS_ENTRY(NAME, PAIRED, EXACT, NORM)                                                           \
    template <int KG, int R, bool FULL>                                                                          \
    __global__ __launch_bounds__(256, MOSS_ROWS_WAVES(PAIRED, NORM, R)) void NAME(const uint16_t* __restrict__ x, const uint4* __restrict__ qw,     \
                                                const uint16_t* __restrict__ sc, const uint8_t* __restrict__ zp, \
                                                uint16_t* __restrict__ y, int G, int n_out, NormArgs na) {      \
        gemv_rows<KG, R, PAIRED, FULL, EXACT, NORM>(x, qw, sc, zp, y, G, n_out, na);                             \
    }
MOSS_ROWS_ENTRY(w4g32_gemv_exact, false, true, 0)
MOSS_ROWS_ENTRY(w4g32_gemv_unrounded, false, false, 0)
MOSS_ROWS_ENTRY(w4g32_gateup_silu_exact, true, true, 0)
MOSS_ROWS_ENTRY(w4g32_gateup_silu_unrounded, true, false, 0)
MOSS_ROWS_ENTRY(w4g32_norm_gemv_exact, false, true, 1)
MOSS_ROWS_ENTRY(w4g32_norm_gemv_unrounded, false, false, 1)
MOSS_ROWS_ENTRY(w4g32_norm_gateup_silu_exact, true, true, 1)
MOSS_ROWS_ENTRY(w4g32_norm_gateup_silu_unrounded, true, false, 1)
MOSS_ROWS_ENTRY(w4g32_addnorm_gemv_exact, false, true, 2)
MOSS_ROWS_ENTRY(w4g32_addnorm_gemv_unrounded, false, false, 2)
MOSS_ROWS_ENTRY(w4g32_addnorm_gateup_silu_exact, true, true, 2)
MOSS_ROWS_ENTRY(w4g32_addnorm_gateup_silu_unrounded, true, false, 2)
#undef MOSS_ROWS_ENTRY

#define MOSS_KSPLIT_ENTRY(NAME, PAIRED, EXACT)                                                                  \
    template <int W, int R>                                                                                     \
    __global__ __launch_bounds__(64 * W) void NAME(const uint16_t* __restrict__ x, const uint4* __restrict__ qw, \
                                                   const uint16_t* __restrict__ sc,                             \
                                                   const uint8_t* __restrict__ zp, uint16_t* __restrict__ y,    \
                                                   int G, int n_out) {                                          \
        gemv_ksplit<W, R, PAIRED, EXACT>(x, qw, sc, zp, y, G, n_out);                                           \
    }
MOSS_KSPLIT_ENTRY(w4g32_gemv_ksplit_exact, false, true)
MOSS_KSPLIT_ENTRY(w4g32_gemv_ksplit_unrounded, false, false)
MOSS_KSPLIT_ENTRY(w4g32_gateup_silu_ksplit_exact, true, true)
MOSS_KSPLIT_ENTRY(w4g32_gateup_silu_ksplit_unrounded, true, false)
#undef MOSS_KSPLIT_ENTRY

template <int KG, int R, bool PAIRED, bool FULL, bool EXACT, int NORM>
constexpr auto rows_kernel() {
    if constexpr (NORM == 0) {
        if constexpr (PAIRED) {
            if constexpr (EXACT) return &w4g32_gateup_silu_exact<KG, R, FULL>;
            else return &w4g32_gateup_silu_unrounded<KG, R, FULL>;
        } else {
            if constexpr (EXACT) return &w4g32_gemv_exact<KG, R, FULL>;
            else return &w4g32_gemv_unrounded<KG, R, FULL>;
        }
    } else if constexpr (NORM == 1) {
        if constexpr (PAIRED) {
            if constexpr (EXACT) return &w4g32_norm_gateup_silu_exact<KG, R, FULL>;
            else return &w4g32_norm_gateup_silu_unrounded<KG, R, FULL>;
        } else {
            if constexpr (EXACT) return &w4g32_norm_gemv_exact<KG, R, FULL>;
            else return &w4g32_norm_gemv_unrounded<KG, R, FULL>;
        }
    } else {
        if constexpr (PAIRED) {
            if constexpr (EXACT) return &w4g32_addnorm_gateup_silu_exact<KG, R, FULL>;
            else return &w4g32_addnorm_gateup_silu_unrounded<KG, R, FULL>;
        } else {
            if constexpr (EXACT) return &w4g32_addnorm_gemv_exact<KG, R, FULL>;
            else return &w4g32_addnorm_gemv_unrounded<KG, R, FULL>;
        }
    }
}

template <int W, int R, bool PAIRED, bool EXACT>
constexpr auto ksplit_kernel() {
    if constexpr (PAIRED) {
        if constexpr (EXACT) return &w4g32_gateup_silu_ksplit_exact<W, R>;
        else return &w4g32_gateup_silu_ksplit_unrounded<W, R>;
    } else {
        if constexpr (EXACT) return &w4g32_gemv_ksplit_exact<W, R>;
        else return &w4g32_gemv_ksplit_unrounded<W, R>;
    }
}

template <bool PAIRED, bool EXACT>
int launch_ksplit(const void* x, const void* qw, const void* sc, const void* zp, void* y, int G, int n_out,
                  int rows, hipStream_t st) {
    const int W = G / 128;
    if (rows <= 0) rows = 4;  // measured on MI355X (K = 12288, N = 4096): 4 rows per wave group in both modes
    const dim3 grid((n_out + rows - 1) / rows);
    const auto* xp = (const uint16_t*)x;
    const auto* qp = (const uint4*)qw;
    const auto* sp = (const uint16_t*)sc;
    const auto* zpp = (const uint8_t*)zp;
    auto* yp = (uint16_t*)y;
#define MOSS_KS(WV, RV)                                                                                      \
    if (W == WV && rows == RV) {                                                                             \
        hipLaunchKernelGGL((ksplit_kernel<WV, RV, PAIRED, EXACT>()), grid, dim3(64 * WV), 0, st, xp, qp, sp, \
                           zpp, yp, G, n_out);                                                               \
        return moss_launch_status();                                                                         \
    }
    MOSS_KS(2, 1) MOSS_KS(2, 2) MOSS_KS(2, 4)
    MOSS_KS(3, 1) MOSS_KS(3, 2) MOSS_KS(3, 4)
    MOSS_KS(4, 1) MOSS_KS(4, 2) MOSS_KS(4, 4)
#undef MOSS_KS
    return (int)hipErrorInvalidValue;
}

template <bool PAIRED, int R, bool EXACT, int NORM>
int launch_rows(const void* x, const void* qw, const void* sc, const void* zp, void* y, int G, int n_out,
                const NormArgs& na, hipStream_t st) {
    const int KG = (G + kWave - 1) / kWave;
    const int waves = (n_out + R - 1) / R;
    const dim3 grid((waves + 3) / 4), block(256);
    const auto* xp = (const uint16_t*)x;
    const auto* qp = (const uint4*)qw;
    const auto* sp = (const uint16_t*)sc;
    const auto* zpp = (const uint8_t*)zp;
    auto* yp = (uint16_t*)y;
    const bool full = (G == kWave * KG) && (KG % 2 == 0);
    switch (KG) {
#define MOSS_KG_CASE(KGV)                                                                                          \
    case KGV:                                                                                                      \
        if constexpr (NORM == 0 || KGV <= 4) {                                                                     \
            if (full)                                                                                              \
                hipLaunchKernelGGL((rows_kernel<KGV, R, PAIRED, (KGV % 2 == 0), EXACT, NORM>()), grid, block, 0, st, \
                                   xp, qp, sp, zpp, yp, G, n_out, na);                                             \
            else                                                                                                   \
                hipLaunchKernelGGL((rows_kernel<KGV, R, PAIRED, false, EXACT, NORM>()), grid, block, 0, st, xp, qp, \
                                   sp, zpp, yp, G, n_out, na);                                                     \
            break;                                                                                                 \
        } else {                                                                                                   \
            return (int)hipErrorInvalidValue;                                                                      \
        }
        MOSS_KG_CASE(1)
        MOSS_KG_CASE(2)
        MOSS_KG_CASE(3)
        MOSS_KG_CASE(4)
        MOSS_KG_CASE(5)
        MOSS_KG_CASE(6)
        MOSS_KG_CASE(7)
        MOSS_KG_CASE(8)
#undef MOSS_KG_CASE
        default: return (int)hipErrorInvalidValue;
    }
    return moss_launch_status();
}

template <bool PAIRED, bool EXACT, int NORM>
int launch_gemv_mode(const void* x, const void* qw, const void* sc, const void* zp, void* y, int G, int n_out,
                     int rows, const NormArgs& na, hipStream_t st) {
    switch (rows) {
        case 1: return launch_rows<PAIRED, 1, EXACT, NORM>(x, qw, sc, zp, y, G, n_out, na, st);
        case 2: return launch_rows<PAIRED, 2, EXACT, NORM>(x, qw, sc, zp, y, G, n_out, na, st);
        case 4: return launch_rows<PAIRED, 4, EXACT, NORM>(x, qw, sc, zp, y, G, n_out, na, st);
        default: return (int)hipErrorInvalidValue;
    }
}

template <bool PAIRED, int NORM>
int launch_gemv(const void* x, const void* qw, const void* sc, const void* zp, void* y, int K, int n_out,
                int rows, int mode, const NormArgs& na, hipStream_t st) {
    const int G = K / 32;
    if (rows < 0 || rows == 3 || rows > 4) return (int)hipErrorInvalidValue;
    if (NORM == 0 && G % 128 == 0 && G >= 256 && G <= 512) {
        if (mode == MOSS_DEQUANT_EXACT) return launch_ksplit<PAIRED, true>(x, qw, sc, zp, y, G, n_out, rows, st);
        if (mode == MOSS_DEQUANT_UNROUNDED) return launch_ksplit<PAIRED, false>(x, qw, sc, zp, y, G, n_out, rows, st);
        return (int)hipErrorInvalidValue;
    }
    // measured on MI355X (K = 4096): 2 rows per wave is best for the exact mode in both roles and
    // every N (N = 24576 / 32802: 12.3 / 15.3 us against 13.6 / 17.2 at 4), except the fused
    // add-RMSNorm form of the 32-head output projection (N ~ 32800: 18.8 us at 4, 20.9 at 2); the
    // unrounded GEMV is as fast at 4 and the unrounded gate||up at 2
    if (rows == 0)
        rows = (G <= 128)
                   ? ((PAIRED || mode == MOSS_DEQUANT_EXACT) ? (!PAIRED && NORM > 0 && n_out >= 24576 ? 4 : 2) : 4)
                   : (G <= 256 ? 2 : 1);
    if (mode == MOSS_DEQUANT_EXACT)
        return launch_gemv_mode<PAIRED, true, NORM>(x, qw, sc, zp, y, G, n_out, rows, na, st);
    if (mode == MOSS_DEQUANT_UNROUNDED)
        return launch_gemv_mode<PAIRED, false, NORM>(x, qw, sc, zp, y, G, n_out, rows, na, st);
    return (int)hipErrorInvalidValue;
}

}  // namespace

// M = 2 .. kMaxTokens tokens through the exact GEMV (one weight stream for all of them); K as the
// single-token GEMV takes it up to 4096 and K = 8192, 12288, 16384.  hipErrorInvalidValue for
// other shapes (the caller then uses another kernel).
int w4g32_gemv_tokens_launch(const void* x, const void* qw, const void* sc, const void* zp, void* y, int M, int K,
                             int N, hipStream_t st) {
    if (K % 64 || N <= 0) return (int)hipErrorInvalidValue;
    const int G = K / 32;
    switch (M) {
        case 2: return launch_tokens_t<2>(x, qw, sc, zp, y, G, N, st);
        case 3: return launch_tokens_t<3>(x, qw, sc, zp, y, G, N, st);
        case 4: return launch_tokens_t<4>(x, qw, sc, zp, y, G, N, st);
        default: return (int)hipErrorInvalidValue;
    }
}

bool w4g32_gemv_tokens_shape(int M, int K) {
    if (M < 2 || M > kMaxTokens || K % 64) return false;
    const int G = K / 32;
    return G <= 128 || (G % 128 == 0 && G <= 512);
}

}  // namespace moss

using namespace moss;

// Largest K the register-resident x slice supports: 8 groups per lane.
static constexpr int kMaxGemvK = 8 * 64 * 32;

MOSS_API int moss_w4g32_gemv(const void* x, const void* qw, const void* sc, const void* zp, void* y, int M, int K,
                             int N, int rows_per_wave, int dequant_mode, void* stream) {
    MOSS_CHECK_ARG(x && qw && sc && zp && y);
    MOSS_CHECK_ARG(M >= 1 && K > 0 && N > 0 && K % 64 == 0 && K <= kMaxGemvK);
    MOSS_CHECK_ARG(MOSS_ALIGNED(x, 16) && MOSS_ALIGNED(qw, 16));
    if (M > 1) {
        MOSS_CHECK_ARG(dequant_mode == MOSS_DEQUANT_EXACT && w4g32_gemv_tokens_shape(M, K));
        return w4g32_gemv_tokens_launch(x, qw, sc, zp, y, M, K, N, (hipStream_t)stream);
    }
    return launch_gemv<false, 0>(x, qw, sc, zp, y, K, N, rows_per_wave, dequant_mode, NormArgs{}, (hipStream_t)stream);
}

MOSS_API int moss_w4g32_gateup_silu(const void* x, const void* qw, const void* sc, const void* zp, void* y, int M,
                                    int K, int N_half, int rows_per_wave, int dequant_mode, void* stream) {
    MOSS_CHECK_ARG(x && qw && sc && zp && y);
    MOSS_CHECK_ARG(M == 1 && K > 0 && N_half > 0 && K % 64 == 0 && K <= kMaxGemvK);
    MOSS_CHECK_ARG(MOSS_ALIGNED(x, 16) && MOSS_ALIGNED(qw, 16));
    return launch_gemv<true, 0>(x, qw, sc, zp, y, K, N_half, rows_per_wave, dequant_mode, NormArgs{},
                                (hipStream_t)stream);
}

MOSS_API int moss_w4g32_norm_gemv(const void* x, const void* res, const void* norm_w, void* sum_out, float eps,
                                  const void* qw, const void* sc, const void* zp, void* y, int K, int N,
                                  int rows_per_wave, int dequant_mode, void* stream) {
    if (int rc = moss_check_norm_args(x, res, norm_w, sum_out, K, eps)) return rc;
    MOSS_CHECK_ARG(qw && sc && zp && y && N > 0 && MOSS_ALIGNED(qw, 16));
    const NormArgs na{(const uint16_t*)res, (const uint16_t*)norm_w, (uint16_t*)sum_out, eps};
    if (res)
        return launch_gemv<false, 2>(x, qw, sc, zp, y, K, N, rows_per_wave, dequant_mode, na, (hipStream_t)stream);
    return launch_gemv<false, 1>(x, qw, sc, zp, y, K, N, rows_per_wave, dequant_mode, na, (hipStream_t)stream);
}

MOSS_API int moss_w4g32_norm_gateup_silu(const void* x, const void* res, const void* norm_w, void* sum_out,
                                         float eps, const void* qw, const void* sc, const void* zp, void* y, int K,
                                         int N_half, int rows_per_wave, int dequant_mode, void* stream) {
    if (int rc = moss_check_norm_args(x, res, norm_w, sum_out, K, eps)) return rc;
    MOSS_CHECK_ARG(qw && sc && zp && y && N_half > 0 && MOSS_ALIGNED(qw, 16));
    const NormArgs na{(const uint16_t*)res, (const uint16_t*)norm_w, (uint16_t*)sum_out, eps};
    if (res)
        return launch_gemv<true, 2>(x, qw, sc, zp, y, K, N_half, rows_per_wave, dequant_mode, na,
                                    (hipStream_t)stream);
    return launch_gemv<true, 1>(x, qw, sc, zp, y, K, N_half, rows_per_wave, dequant_mode, na, (hipStream_t)stream);
}
