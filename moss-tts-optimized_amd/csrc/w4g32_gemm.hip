// Prefill GEMM on MFMA: Y[M, N] = X[M, K] . W[N, K]^T, bf16 in/out, fp32 accumulate, for
// INT4 group-32 weights (row-packed) and for FP8 E4M3 weights with fp32 row scales.
//
// INT4: the reference keeps bf16 weights for prefill (src/moss_tts/_runtime/llm.py:29,84,130);
// its dequant-then-matmul (src/moss_tts/calibration.py:185-188) is the contract here.  Every
// weight is dequantized bit-exactly, bf16_rne((q - z) * s) as in
// src/moss_tts/_runtime/calibrated_quant.py:41-42, and then multiplied on the matrix cores
// (v_mfma_f32_32x32x16_bf16).
// FP8: every e4m3 value is a bf16 value, so the B-tile producer converts exactly
// (v_cvt_scalef32_pk_bf16_fp8, scale 1) and the row scale multiplies the fp32 sum in the
// epilogue (src/moss_tts/_runtime/fused_mlp.py:20-21).  The fp8 MFMA forms are not used:
// they would round the bf16 activations to e4m3 as well.
//
// INT4 takes the register-weight tile wherever its shape conditions hold (reg_tile_shape): the
// dequantized weights are the MFMA's A operand straight from the registers that dequantize them,
// and only the activations are staged in LDS (w4g32_gemm_t_kernel up to 64 tokens per tile;
// w4g32_gemm_tdma_kernel, whose activations go from global memory to LDS without registers, for
// 128).  FP8, other INT4 shapes and misaligned scale or zero-point pointers take the LDS tiles:
//
// LDS tiles: BM x BN outputs (BM, BN in {64, 128}) per 256-thread workgroup, 2 x 2 waves of
// (BM/2) x (BN/2), K in steps of 64 (two quantization groups).  Pipeline: two LDS buffers and
// S register stages (stages_for); while step st is multiplied from one LDS buffer and step st + 1
// is converted into the other, the global loads of step st + S are issued, so every load has
// S - 1 steps of MFMA work to arrive (one barrier per step).
// Split-K (SPLIT): workgroup z of a tile covers K range [z K/S, (z+1) K/S) and stores fp32
// partial sums; gemm_reduce adds them in z order (deterministic) and applies the epilogue.
// It is used when the tiles alone cannot fill the 256 CUs (small M).
// Tile order: logical tiles are n-major with the M tiles of one N tile adjacent, and the
// workgroup id is remapped so that consecutive logical tiles run on the same XCD (workgroups
// are dealt to the 8 XCDs round-robin), so a weight tile is fetched into one L2.
#include "common.h"

#include <mutex>
#include <type_traits>

namespace moss {
namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

constexpr int kBK = 64;
constexpr int kPad = 8;  // bf16 padding per LDS row: breaks the 128-byte bank period
constexpr int kLds = kBK + kPad;
constexpr int kXcds = 8;
// Register stages of the global-load pipeline: 4, or 2 for the 128 x 128 tile, whose 64
// accumulators leave room for two stages at two waves per SIMD.
template <int BM, int BN>
constexpr int stages_for() { return BM == 128 && BN == 128 ? 2 : 4; }

enum WeightFormat { kInt4G32 = 0, kFp8E4M3 = 1 };

typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));

// Per-thread share of one K step: BM rows x 64 activations (BM / 32 x 16 B per thread) and one
// piece of the BN x 64 weight tile.  The weight tile is 2 BN (row, 32-wide half) units; with
// BN = 64 two threads share a unit (TPU = 2), each taking half of it.
template <int BM, int BN>
struct StepRegs {
    static constexpr int TPU = 256 / (2 * BN), WPT = 4 / TPU;  // threads per unit; INT4 code words per thread
    u32x4_t x[BM / 32];
    uint32_t w[2 * WPT];  // INT4: WPT words of codes (8 codes each); FP8: 2 WPT words of e4m3 bytes
    uint32_t s, z, zsh;   // INT4: the group's scale bits, and the byte holding its zero point at bit zsh
};

// Per-thread addressing, fixed for a workgroup: the thread's activation row and weight row.
template <int BM, int BN>
struct StepAddr {
    const uint16_t* x[BM / 32];  // chunk t % 8 of activation rows t / 8 + 32 c (see step_addr)
    size_t wrow;        // weight row n (clamped)
    int half, sub;      // which 32-wide half of the step, which part of it
};

// Out-of-range rows and columns load the last valid row / column instead (addresses are clamped
// here): rows of X and columns of W are independent in the product, and those outputs are never
// stored.  Every thread then issues the same loads.  Activations: load c moves 16-byte chunk
// t % 8 of row t / 8 + 32 c, so the eight threads of a row cover its 128 bytes of the step and
// an instruction touches 16 64-byte segments (memory requests are counted per segment).
template <int BM, int BN>
__device__ __forceinline__ StepAddr<BM, BN> step_addr(const uint16_t* __restrict__ X, int M, int N, int K, int m0,
                                                      int n0, int tid) {
    constexpr int CH = BM / 32, TPU = StepRegs<BM, BN>::TPU;
    StepAddr<BM, BN> a;
#pragma unroll
    for (int c = 0; c < CH; ++c) a.x[c] = X + (size_t)min(m0 + (tid >> 3) + 32 * c, M - 1) * K + 8 * (tid & 7);
    const int unit = tid / TPU;
    a.wrow = (size_t)min(n0 + (unit >> 1), N - 1);
    a.half = unit & 1;
    a.sub = tid % TPU;
    return a;
}

template <int BM, int BN>
__device__ __forceinline__ void load_a(StepRegs<BM, BN>& r, const StepAddr<BM, BN>& a, int k0) {
    constexpr int CH = BM / 32;
#pragma unroll
    for (int c = 0; c < CH; ++c) r.x[c] = __builtin_bit_cast(u32x4_t, *reinterpret_cast<const uint4*>(a.x[c] + k0));
}

template <int BM, int BN, int FMT>
__device__ __forceinline__ void load_b(StepRegs<BM, BN>& r, const StepAddr<BM, BN>& a,
                                       const uint4* __restrict__ qw, const uint16_t* __restrict__ sc,
                                       const uint8_t* __restrict__ zp, int K, int G, int k0) {
    constexpr int WPT = StepRegs<BM, BN>::WPT;
    if constexpr (FMT == kInt4G32) {
        const int g = (k0 >> 5) + a.half;
        int zb;
        zero_loc(g, G, zb, r.zsh);
        const uint32_t* codes = reinterpret_cast<const uint32_t*>(qw + a.wrow * G + g) + WPT * a.sub;
        if constexpr (WPT == 4) {
            const uint4 v = *reinterpret_cast<const uint4*>(codes);
            r.w[0] = v.x; r.w[1] = v.y; r.w[2] = v.z; r.w[3] = v.w;
        } else {
            const uint2 v = *reinterpret_cast<const uint2*>(codes);
            r.w[0] = v.x; r.w[1] = v.y;
        }
        r.s = sc[a.wrow * G + g];
        r.z = zp[a.wrow * (G >> 1) + zb];  // raw byte: the nibble is taken where it is used
    } else {
        // 32 e4m3 bytes per unit: 8 words, 2 WPT of them per thread
        const uint32_t* p = reinterpret_cast<const uint32_t*>(reinterpret_cast<const uint8_t*>(qw) + a.wrow * K + k0 +
                                                              32 * a.half) + 2 * WPT * a.sub;
        const uint4 v0 = reinterpret_cast<const uint4*>(p)[0];
        r.w[0] = v0.x; r.w[1] = v0.y; r.w[2] = v0.z; r.w[3] = v0.w;
        if constexpr (WPT == 4) {
            const uint4 v1 = reinterpret_cast<const uint4*>(p)[1];
            r.w[4] = v1.x; r.w[5] = v1.y; r.w[6] = v1.z; r.w[7] = v1.w;
        }
    }
}

template <int BM, int BN, int FMT>
__device__ __forceinline__ void load_step(StepRegs<BM, BN>& r, const StepAddr<BM, BN>& a,
                                          const uint4* __restrict__ qw, const uint16_t* __restrict__ sc,
                                          const uint8_t* __restrict__ zp, int K, int G, int k0) {
    load_a<BM, BN>(r, a, k0);
    load_b<BM, BN, FMT>(r, a, qw, sc, zp, K, G, k0);
}

// Keeps the scheduler from moving instructions across this point: the loads of a pipeline stage
// stay where they are issued instead of being sunk next to their first use (which would shrink
// the prefetch distance to nothing); the compiler still places the waits before each use.
__device__ __forceinline__ void pin() { __builtin_amdgcn_sched_barrier(0); }

// Two e4m3 codes (bytes 2p, 2p+1 of a word pair) -> bf16 pair; exact: every e4m3 value is a bf16 value.
template <bool HI>
__device__ __forceinline__ uint32_t fp8x2_to_bf16x2(uint32_t w) {
    return __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w, 1.0f, HI));
}

template <int BM, int BN>
__device__ __forceinline__ void store_a(const StepRegs<BM, BN>& r, uint16_t (*As)[kLds], int tid) {
    constexpr int CH = BM / 32;
#pragma unroll
    for (int c = 0; c < CH; ++c) *reinterpret_cast<u32x4_t*>(&As[(tid >> 3) + 32 * c][8 * (tid & 7)]) = r.x[c];
}

template <int BM, int BN, int FMT>
__device__ __forceinline__ void store_b(const StepRegs<BM, BN>& r, const StepAddr<BM, BN>& ad, uint16_t (*Bs)[kLds],
                                        int tid) {
    constexpr int TPU = StepRegs<BM, BN>::TPU, WPT = StepRegs<BM, BN>::WPT;
    const int row = (tid / TPU) >> 1;
    constexpr int NOUT = 4 * WPT;  // bf16 pairs per thread (32 / TPU weights)
    uint32_t out[NOUT];
    if constexpr (FMT == kFp8E4M3) {
#pragma unroll
        for (int c = 0; c < 2 * WPT; ++c) {
            out[2 * c] = fp8x2_to_bf16x2<false>(r.w[c]);
            out[2 * c + 1] = fp8x2_to_bf16x2<true>(r.w[c]);
        }
    } else {
        const MixedUnpack mu = make_mixed_unpack();
        const GroupDequant gd = group_dequant(r.s, (r.z >> r.zsh) & 15u);
#pragma unroll
        for (int j = 0; j < WPT; ++j) {
            uint32_t o[4];
            dequant_word_mixed(r.w[j], mu, gd.s_lo, gd.s_hi, gd.s, gd.bias_bf16, gd.bias_f16, o);
#pragma unroll
            for (int i = 0; i < 4; ++i) out[4 * j + i] = o[i];
        }
    }
    uint4* b = reinterpret_cast<uint4*>(&Bs[row][32 * ad.half + (32 / TPU) * ad.sub]);
#pragma unroll
    for (int c = 0; c < NOUT / 4; ++c) b[c] = make_uint4(out[4 * c], out[4 * c + 1], out[4 * c + 2], out[4 * c + 3]);
}

template <int BM, int BN, int FMT>
__device__ __forceinline__ void store_step(const StepRegs<BM, BN>& r, const StepAddr<BM, BN>& ad,
                                           uint16_t (*As)[kLds], uint16_t (*Bs)[kLds], int tid) {
    store_a<BM, BN>(r, As, tid);
    store_b<BM, BN, FMT>(r, ad, Bs, tid);
}

template <int BM, int BN>
__device__ __forceinline__ void mfma_step(const uint16_t (*As)[kLds], const uint16_t (*Bs)[kLds],
                                          f32x16_t (&acc)[BM / 64][BN / 64], int lane, int wm, int wn) {
    constexpr int TM = BM / 64, TN = BN / 64;  // 32 x 32 MFMA tiles per wave
#pragma unroll
    for (int kk = 0; kk < kBK / 16; ++kk) {
        const int kc = 16 * kk + 8 * (lane >> 5);
        bf16x8_t a[TM], b[TN];
#pragma unroll
        for (int i = 0; i < TM; ++i)
            a[i] = *reinterpret_cast<const bf16x8_t*>(&As[(BM / 2) * wm + 32 * i + (lane & 31)][kc]);
#pragma unroll
        for (int j = 0; j < TN; ++j)
            b[j] = *reinterpret_cast<const bf16x8_t*>(&Bs[(BN / 2) * wn + 32 * j + (lane & 31)][kc]);
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
            for (int j = 0; j < TN; ++j)
                acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[i], b[j], acc[i][j], 0, 0, 0);
    }
}

// FMT == kFp8E4M3: qw is e4m3 [N, K] (row-major bytes), `row_scale` fp32 [N] or null.
// SPLIT: `part` is fp32 [S, M, N]; gridDim.y = S.  TAIL: the K steps of one workgroup need not
// be a multiple of the stage count.
template <int BM, int BN, int FMT, bool SPLIT, bool TAIL>
__global__ __launch_bounds__(256) void w4g32_gemm_kernel(const uint16_t* __restrict__ X, const uint4* __restrict__ qw,
                                                         const uint16_t* __restrict__ sc,
                                                         const uint8_t* __restrict__ zp, uint16_t* __restrict__ Y,
                                                         float* __restrict__ part, int M, int N, int K,
                                                         const float* __restrict__ row_scale) {
    static_assert((BM == 64 || BM == 128) && (BN == 64 || BN == 128), "tile");
    constexpr int TM = BM / 64, TN = BN / 64;
    __shared__ __attribute__((aligned(16))) uint16_t As[2][BM][kLds];
    __shared__ __attribute__((aligned(16))) uint16_t Bs[2][BN][kLds];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    // XCD-aware logical tile (n-major, M tiles of one N tile adjacent)
    const int mt = (M + BM - 1) / BM, tiles = gridDim.x;
    int tile = blockIdx.x;
    if (tiles % kXcds == 0) tile = (blockIdx.x % kXcds) * (tiles / kXcds) + blockIdx.x / kXcds;
    const int m0 = (tile % mt) * BM, n0 = (tile / mt) * BN;
    const int G = K >> 5;
    const int steps = K / kBK / gridDim.y;
    const int kbase = blockIdx.y * steps * kBK;

    f32x16_t acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j)
#pragma unroll
            for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.f;

    constexpr int kStages_ = stages_for<BM, BN>();
    // register stage i % kStages_ holds step i; kStages_ is even, so step i's LDS buffer is i % 2.
    // Every sub-step issues one stage of loads (steps past the end load the last step again),
    // so the stage consumed next has (kStages_ - 1) stages of loads issued after it.
    static_assert(kStages_ % 2 == 0, "stages");
    const StepAddr<BM, BN> ad = step_addr<BM, BN>(X, M, N, K, m0, n0, tid);
    StepRegs<BM, BN> r[kStages_];
#pragma unroll
    for (int i = 0; i < kStages_; ++i) load_step<BM, BN, FMT>(r[i], ad, qw, sc, zp, K, G, kbase + min(i, steps - 1) * kBK);
    pin();
    store_step<BM, BN, FMT>(r[0], ad, As[0], Bs[0], tid);
    __syncthreads();
    // whole trips of kStages_ steps (at the very last step the store writes a copy of that step
    // into the idle buffer, which is never read), then, with TAIL, the remaining steps with guards
    int st = 0;
    for (; st + kStages_ <= steps; st += kStages_) {
#pragma unroll
        for (int i = 0; i < kStages_; ++i) {
            load_step<BM, BN, FMT>(r[i], ad, qw, sc, zp, K, G, kbase + min(st + i + kStages_, steps - 1) * kBK);
            pin();
            mfma_step<BM, BN>(As[i % 2], Bs[i % 2], acc, lane, wm, wn);
            store_step<BM, BN, FMT>(r[(i + 1) % kStages_], ad, As[(i + 1) % 2], Bs[(i + 1) % 2], tid);
            __syncthreads();
        }
    }
#pragma unroll
    for (int i = 0; i < kStages_ - 1; ++i) {
        const int s = st + i;
        if (TAIL && s < steps) {  // uniform
            load_step<BM, BN, FMT>(r[i], ad, qw, sc, zp, K, G, kbase + (steps - 1) * kBK);
            pin();
            mfma_step<BM, BN>(As[i % 2], Bs[i % 2], acc, lane, wm, wn);
            if (s + 1 < steps) store_step<BM, BN, FMT>(r[(i + 1) % kStages_], ad, As[(i + 1) % 2], Bs[(i + 1) % 2], tid);
            __syncthreads();
        }
    }
    // C layout of a 32 x 32 tile: lane l, element e -> row 8 (e / 4) + 4 (l / 32) + e % 4, column l % 32
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) {
            const int n = n0 + (BN / 2) * wn + 32 * j + (lane & 31);
            if (n >= N) continue;
            // FP8: the per-row scale multiplies the finished sum (src/moss_tts/_runtime/fused_mlp.py:20-21)
            const float rs = (!SPLIT && FMT == kFp8E4M3 && row_scale) ? row_scale[n] : 1.0f;
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                const int m = m0 + (BM / 2) * wm + 32 * i + 8 * (e >> 2) + 4 * (lane >> 5) + (e & 3);
                if (m >= M) continue;
                if constexpr (SPLIT)
                    part[((size_t)blockIdx.y * M + m) * N + n] = acc[i][j][e];
                else
                    Y[(size_t)m * N + n] = f32_to_bf16(FMT == kFp8E4M3 ? acc[i][j][e] * rs : acc[i][j][e]);
            }
        }
}

// Weight-stationary-in-registers INT4 tile (Y^T = W X^T): the dequantized weights are the MFMA's
// A operand, formed in the registers of the lane that feeds them, so they never pass through
// LDS; only the activation tile does.  A workgroup covers 128 weight rows and
// BM = 32 JT tokens: wave w owns weight rows n0 + 32 w .. + 31 and every token (JT MFMA tiles
// of 32 x 32).  In a K step of 64, lane l takes row n0 + 32 w + (l & 31) and the 32-wide half
// (l >> 5) of the step: its 32 weights are the A operands of the step's 4 MFMAs (8 per MFMA),
// and MFMA kk meets the activations x[m][32 (l >> 5) + 8 kk .. + 8] of the same lane, so both
// operands walk K in the same order: one group of 32 codes (16 bytes) per lane and step,
// dequantized bit-exactly.  (FP8 weights measured slower in this tile than in the LDS tiles at
// M <= 128 and take those.)
// Vector-memory requests are counted per 64-byte segment an instruction touches, so every load
// is shaped to touch few: eight consecutive threads copy one token row's 128 bytes of a step, and
// the scales and zero points of a row come once per block of kTs steps (8 groups: 16 bytes
// of scales, 8 zero bytes that all hold the same nibble half when the row's last 128-group
// chunk is a multiple of 16 groups long).  Weights travel kTs steps ahead (HBM), activations
// two steps ahead (mostly L2 hits), scales and zeros one block ahead.
constexpr int kTs = 4;

struct TBlock {
    uint4 s;   // scales of groups 8b .. 8b + 7
    uint2 z;   // zero bytes of those groups
    uint32_t zsh;
};

// SPLIT: gridDim.y workgroups share a tile, each summing a contiguous K range of whole blocks
// into fp32 partials part[blockIdx.y, M, N], reduced by gemm_reduce.
template <int JT, bool SPLIT>
__global__ __launch_bounds__(256) void w4g32_gemm_t_kernel(const uint16_t* __restrict__ X, const uint4* __restrict__ qw,
                                                           const uint16_t* __restrict__ sc,
                                                           const uint8_t* __restrict__ zp, uint16_t* __restrict__ Y,
                                                           float* __restrict__ part, int M, int N, int K) {
    constexpr int BN = 128, BM = 32 * JT;
    __shared__ __attribute__((aligned(16))) uint16_t Xs[2][BM][kLds];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int mt = (M + BM - 1) / BM, tiles = gridDim.x;
    int tile = blockIdx.x;
    if (tiles % kXcds == 0) tile = (blockIdx.x % kXcds) * (tiles / kXcds) + blockIdx.x / kXcds;
    const int m0 = (tile % mt) * BM, n0 = (tile / mt) * BN;
    const int G = K >> 5, steps = SPLIT ? K / kBK / gridDim.y : K / kBK;
    const int kbase = SPLIT ? blockIdx.y * steps * kBK : 0;  // a multiple of kTs steps (8 groups)
    // activation copy: thread t moves 16-byte chunk t % 8 of token rows t / 8 + 32 c, c < JT
    // (rows clamped; those outputs are not stored)
    const int xc = tid & 7, xr = tid >> 3;
    const uint16_t* xrow[JT];
#pragma unroll
    for (int c = 0; c < JT; ++c) xrow[c] = X + (size_t)min(m0 + xr + 32 * c, M - 1) * K + kbase + 8 * xc;
    // weights: this lane's row and 32-wide half of the step
    const int half = lane >> 5;
    const size_t wrow = (size_t)min(n0 + 32 * wave + (lane & 31), N - 1);

    auto load_x = [&](u32x4_t (&x)[JT], int k0) {
#pragma unroll
        for (int c = 0; c < JT; ++c) x[c] = __builtin_bit_cast(u32x4_t, *reinterpret_cast<const uint4*>(xrow[c] + k0));
    };
    auto load_w = [&](uint4& w, int k0) { w = qw[wrow * G + ((kbase + k0) >> 5) + half]; };
    auto load_blk = [&](TBlock& t, int blk) {
        const int g = (kbase >> 5) + 8 * blk;
        int zb;
        zero_loc(g, G, zb, t.zsh);
        t.s = *reinterpret_cast<const uint4*>(sc + wrow * G + g);
        t.z = *reinterpret_cast<const uint2*>(zp + wrow * (G >> 1) + zb);
    };
    auto store_x = [&](const u32x4_t (&x)[JT], uint16_t (*xs)[kLds]) {
#pragma unroll
        for (int c = 0; c < JT; ++c) *reinterpret_cast<u32x4_t*>(&xs[xr + 32 * c][8 * xc]) = x[c];
    };

    f32x16_t acc[JT];
#pragma unroll
    for (int j = 0; j < JT; ++j)
#pragma unroll
        for (int e = 0; e < 16; ++e) acc[j][e] = 0.f;

    const int blocks = steps / kTs;
    uint4 cw[kTs];
    u32x4_t xv[2][JT];
    TBlock cur, nxt;
    load_blk(cur, 0);
    load_blk(nxt, min(1, blocks - 1));
#pragma unroll
    for (int i = 0; i < kTs; ++i) load_w(cw[i], min(i, steps - 1) * kBK);
    load_x(xv[0], 0);
    load_x(xv[1], min(1, steps - 1) * kBK);
    pin();
    store_x(xv[0], Xs[0]);
    __syncthreads();
    const MixedUnpack mu = make_mixed_unpack();
    for (int blk = 0; blk < blocks; ++blk) {
        const int st = blk * kTs;
#pragma unroll
        for (int i = 0; i < kTs; ++i) {
            const int s = st + i;
            // all activation operands of the step first: their LDS latency is hidden behind the
            // dequantization below instead of being exposed before each MFMA
            const uint16_t (*xs)[kLds] = Xs[i % 2];
            bf16x8_t b[4][JT];
#pragma unroll
            for (int kk = 0; kk < 4; ++kk)
#pragma unroll
                for (int j = 0; j < JT; ++j)
                    b[kk][j] = *reinterpret_cast<const bf16x8_t*>(&xs[32 * j + (lane & 31)][32 * half + 8 * kk]);
            pin();
            // this step's A operands (group 8 blk + 2 i + half of this lane's row), in registers
            uint32_t wf[4][4];
            {
                const uint32_t sw = i == 0 ? cur.s.x : i == 1 ? cur.s.y : i == 2 ? cur.s.z : cur.s.w;
                const uint32_t zw = i < 2 ? cur.z.x : cur.z.y;
                const uint32_t zq = (zw >> (8 * (2 * (i & 1) + half) + cur.zsh)) & 15u;
                const GroupDequant gd = group_dequant(sw >> (16 * half), zq);
                const uint32_t words[4] = {cw[i].x, cw[i].y, cw[i].z, cw[i].w};
#pragma unroll
                for (int kk = 0; kk < 4; ++kk)
                    dequant_word_mixed(words[kk], mu, gd.s_lo, gd.s_hi, gd.s, gd.bias_bf16, gd.bias_f16, wf[kk]);
            }
            pin();
            // slot i of the code ring is free once dequantized: codes of step s + kTs into it
            load_w(cw[i], min(s + kTs, steps - 1) * kBK);
            if (i == kTs - 1) {
                cur = nxt;
                load_blk(nxt, min(blk + 2, blocks - 1));
            }
            // the next step's activations into the other buffer, which every wave finished reading
            // before the previous barrier (after the last step this writes clamped data nobody reads);
            // their register slot then takes step s + 2
            store_x(xv[(i + 1) % 2], Xs[(i + 1) % 2]);
            load_x(xv[i % 2], min(s + 2, steps - 1) * kBK);
            pin();
#pragma unroll
            for (int kk = 0; kk < 4; ++kk) {
                const bf16x8_t a = __builtin_bit_cast(bf16x8_t, u32x4_t{wf[kk][0], wf[kk][1], wf[kk][2], wf[kk][3]});
#pragma unroll
                for (int j = 0; j < JT; ++j) acc[j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b[kk][j], acc[j], 0, 0, 0);
            }
            __syncthreads();
        }
    }
    // C[n][m] of the 32 x 32 tile (n0 + 32 wave, m0 + 32 j): lane l, element e -> n row
    // 8 (e / 4) + 4 (l / 32) + e % 4, m column l % 32; the four e of a quad are consecutive n
    // (N % 4 == 0: a quad is all in range or all out)
#pragma unroll
    for (int j = 0; j < JT; ++j) {
        const int m = m0 + 32 * j + (lane & 31);
        if (m >= M) continue;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const int n = n0 + 32 * wave + 8 * q + 4 * (lane >> 5);
            if (n >= N) continue;
            const float v0 = acc[j][4 * q], v1 = acc[j][4 * q + 1], v2 = acc[j][4 * q + 2], v3 = acc[j][4 * q + 3];
            if constexpr (SPLIT) {
                *reinterpret_cast<float4*>(part + ((size_t)blockIdx.y * M + m) * N + n) = make_float4(v0, v1, v2, v3);
            } else {
                uint2 o;
                o.x = pack_bf16x2(v0, v1);
                o.y = pack_bf16x2(v2, v3);
                *reinterpret_cast<uint2*>(Y + (size_t)m * N + n) = o;
            }
        }
    }
}

// The 128-token register-weight tile (M > 64) with the activations copied from global memory
// straight into LDS (global_load_lds_dwordx4: lane i of an instruction writes bytes 16 i .. + 15
// of a 1 KiB span), so no registers stage them and no LDS stores are issued: 150-152 VGPRs, three
// workgroups per CU (768 gate||up tiles at M = 512 run in one round instead of 1.5).  Weights,
// operands, MFMA order and results are those of w4g32_gemm_t_kernel<4, SPLIT>, bit for bit.
// LDS layout: two buffers of 128 token rows x 128 bytes (one K step), chunk c (8 bf16) of row r
// stored at position c ^ (r & 7) ^ ((r >> 3) & 1): the 16 lanes that read one chunk of 16
// consecutive rows in one LDS cycle (64 banks) hit 16 different 16-byte bank groups (r & 7 alone
// pairs rows r and r + 8 on the same banks: 4 conflict cycles per read, by counters); the eight
// lanes per row of a copy instruction still read that row's 128 contiguous bytes.  The buffers
// are distinct variables, which lets the compiler see that reading one does not wait for the copy
// into the other.
// Step s: copy step s + 1 into the other buffer, multiply step s, load the codes of step s + kTs
// (and the next block's scales and zeros after a block's last step), then wait until this wave's
// copy has landed -- at most the loads issued after it still outstanding (vector memory requests
// complete in order) -- and meet the other waves at the barrier.  The waits are explicit because
// the compiler only knows that a copy must land before this wave reads it, not before other waves
// do.  qw, sc and zp carry no __restrict__, so the compiler barriers (asm memory clobbers) keep
// those loads in program order around the copies and the waits; the block loop runs in pairs so
// that every load lands in the register it is read from (a register copy would wait for it).
__device__ __forceinline__ void cbar() { asm volatile("" ::: "memory"); }

// s_waitcnt vmcnt(n) lgkmcnt(0) (expcnt not waited): vmcnt bits 3:0 and 15:14, expcnt 6:4,
// lgkmcnt 11:8
#define MOSS_WAIT_VM(n) __builtin_amdgcn_s_waitcnt(((n) & 15) | (((n) >> 4) << 14) | (7 << 4))

// SILU (unsplit only): the weights hold 2 N rows, gate rows then up rows, and Y [M, N] receives
// bf16(bf16(silu(g)) * u): a workgroup takes gate rows n0 .. n0 + 63 (waves 0, 1) and the up rows
// of the same outputs (waves 2, 3); each wave pair hands half of its bf16 results to the other
// through LDS, so all four waves evaluate the SiLU.  Equal bit for bit to the unsplit GEMM of all
// 2 N rows followed by moss_silu_mul.
// QKR (unsplit only): the QKV projection of the prompt pass with the q/k head RMSNorm + RoPE and
// the K/V cache write as its epilogue (N = 48 heads of 128: 32 query, 8 key, 8 value heads, one
// head per 128-wide tile); Y receives the query heads [M, 32, 128].  Equal bit for bit to the
// unsplit GEMM followed by moss_qk_norm_rope_kv with cos/sin rows taken by position.
struct QkRope {
    const uint16_t* q_weight;  // [128] head RMSNorm weights
    const uint16_t* k_weight;
    const uint16_t* cos_t;  // [L, 128], row = position
    const uint16_t* sin_t;
    uint16_t* k_cache;  // [8, L, 128]
    uint16_t* v_cache;
    const int64_t* positions;  // [M], clamped into 0 .. L - 1
    int L;
    float eps;
};

template <bool SPLIT, bool SILU = false, bool QKR = false>
__global__ __launch_bounds__(256, 3) void w4g32_gemm_tdma_kernel(const uint16_t* __restrict__ X, const uint4* qw,
                                                              const uint16_t* sc, const uint8_t* zp,
                                                              uint16_t* __restrict__ Y, float* __restrict__ part,
                                                              int M, int N, int K, QkRope qr) {
    static_assert(!(SPLIT && (SILU || QKR)) && !(SILU && QKR), "the epilogues need whole sums");
    constexpr int BN = SILU ? 64 : 128, BM = 128, JT = 4;
    __shared__ __attribute__((aligned(1024))) uint16_t Xa[BM * kBK];
    __shared__ __attribute__((aligned(1024))) uint16_t Xb[BM * kBK];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int mt = (M + BM - 1) / BM, tiles = gridDim.x;
    int tile = blockIdx.x;
    if (tiles % kXcds == 0) tile = (blockIdx.x % kXcds) * (tiles / kXcds) + blockIdx.x / kXcds;
    const int m0 = (tile % mt) * BM, n0 = (tile / mt) * BN;
    const int G = K >> 5, steps = SPLIT ? K / kBK / gridDim.y : K / kBK;
    const int kbase = SPLIT ? blockIdx.y * steps * kBK : 0;  // a multiple of kTs steps (8 groups)
    // copy instruction c of wave w fills rows 8 (4 w + c) .. + 7; lane i writes position i & 7 of
    // row r = 8 (4 w + c) + i / 8, i.e. chunk (i & 7) ^ (r & 7) ^ ((r >> 3) & 1) of it, with
    // r & 7 = (i >> 3) & 7 and (r >> 3) & 1 = c & 1 (rows past M copy row M - 1; those outputs
    // are not stored)
    const uint16_t* xsrc[4];
#pragma unroll
    for (int c = 0; c < 4; ++c) {
        const int r = 8 * (4 * wave + c) + (lane >> 3);
        xsrc[c] = X + (size_t)min(m0 + r, M - 1) * K + kbase + 8 * ((lane & 7) ^ ((lane >> 3) & 7) ^ (c & 1));
    }
    auto copy_x = [&](uint16_t* buf, int k0) {
#pragma unroll
        for (int c = 0; c < 4; ++c) __builtin_amdgcn_global_load_lds(xsrc[c] + k0, buf + 512 * (4 * wave + c), 16, 0, 0);
    };
    // operand kk of token tile j: row 32 j + (l & 31), chunk 4 half + kk of the step
    const int half = lane >> 5;
    const int swz = (lane & 7) ^ ((lane >> 3) & 1);
    uint32_t roff[4];
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) roff[kk] = 128u * (uint32_t)(lane & 31) + 16u * (uint32_t)((4 * half + kk) ^ swz);
    // this lane's weight row (SILU: waves 2 and 3 take the up rows, N further on)
    const int wn = SILU ? n0 + 32 * (wave & 1) + (lane & 31) : n0 + 32 * wave + (lane & 31);
    const size_t wrow = (size_t)min(wn, N - 1) + (SILU && wave >= 2 ? (size_t)N : 0);
    auto load_w = [&](uint4& w, int k0) { w = qw[wrow * G + ((kbase + k0) >> 5) + half]; };
    auto load_blk = [&](TBlock& t, int blk) {
        const int g = (kbase >> 5) + 8 * blk;
        int zb;
        zero_loc(g, G, zb, t.zsh);
        t.s = *reinterpret_cast<const uint4*>(sc + wrow * G + g);
        t.z = *reinterpret_cast<const uint2*>(zp + wrow * (G >> 1) + zb);
    };

    f32x16_t acc[JT];
#pragma unroll
    for (int j = 0; j < JT; ++j)
#pragma unroll
        for (int e = 0; e < 16; ++e) acc[j][e] = 0.f;

    const int blocks = steps / kTs;
    uint4 cw[kTs];
    TBlock tb[2];  // block b's scales and zeros in tb[b & 1]
    copy_x(Xa, 0);
    cbar();
    load_blk(tb[0], 0);
    load_blk(tb[1], min(1, blocks - 1));
#pragma unroll
    for (int i = 0; i < kTs; ++i) load_w(cw[i], min(i, steps - 1) * kBK);
    cbar();
    MOSS_WAIT_VM(0);
    __builtin_amdgcn_s_barrier();
    cbar();
    const MixedUnpack mu = make_mixed_unpack();
    // I: step within the block, P: which tb holds the block's scales, LAST: the last block, whose
    // refills are never read (the compiler drops them, so its waits count nothing after the copy)
    auto step = [&](auto ic, auto pc, auto lc, int blk, const uint16_t* rd, uint16_t* wr) {
        constexpr int i = decltype(ic)::value, P = decltype(pc)::value;
        constexpr bool LAST = decltype(lc)::value;
        const TBlock& cur = tb[P];
        const int s = blk * kTs + i;
        copy_x(wr, min(s + 1, steps - 1) * kBK);  // the last step's copy (unread) is drained below
        cbar();
        const uint32_t sw = i == 0 ? cur.s.x : i == 1 ? cur.s.y : i == 2 ? cur.s.z : cur.s.w;
        const uint32_t zw = i < 2 ? cur.z.x : cur.z.y;
        const uint32_t zq = (zw >> (8 * (2 * (i & 1) + half) + cur.zsh)) & 15u;
        const GroupDequant gd = group_dequant(sw >> (16 * half), zq);
        const char* xs = reinterpret_cast<const char*>(rd);
#pragma unroll
        for (int kk = 0; kk < 4; ++kk) {
            bf16x8_t b[JT];
#pragma unroll
            for (int j = 0; j < JT; ++j) b[j] = *reinterpret_cast<const bf16x8_t*>(xs + roff[kk] + 4096 * j);
            const uint32_t wd = kk == 0 ? cw[i].x : kk == 1 ? cw[i].y : kk == 2 ? cw[i].z : cw[i].w;
            uint32_t wf[4];
            dequant_word_mixed(wd, mu, gd.s_lo, gd.s_hi, gd.s, gd.bias_bf16, gd.bias_f16, wf);
            const bf16x8_t a = __builtin_bit_cast(bf16x8_t, u32x4_t{wf[0], wf[1], wf[2], wf[3]});
#pragma unroll
            for (int j = 0; j < JT; ++j) acc[j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b[j], acc[j], 0, 0, 0);
        }
        pin();
        // code slot i, and after the block's last step its scales, are free: refill them
        load_w(cw[i], min(s + kTs, steps - 1) * kBK);
        if (i == kTs - 1) load_blk(tb[P], min(blk + 2, blocks - 1));
        cbar();
        if (LAST) MOSS_WAIT_VM(0);
        else if (i == kTs - 1) MOSS_WAIT_VM(3);  // one code load, two block loads after the copy
        else MOSS_WAIT_VM(1);                    // one code load after the copy
        __builtin_amdgcn_s_barrier();
        cbar();
    };
    using S0 = std::integral_constant<int, 0>;
    using S1 = std::integral_constant<int, 1>;
    using S2 = std::integral_constant<int, 2>;
    using S3 = std::integral_constant<int, 3>;
    using No = std::false_type;
    using Yes = std::true_type;
    int blk = 0;
    for (; blk + 1 < blocks; blk += 2) {
        step(S0{}, S0{}, No{}, blk, Xa, Xb);
        step(S1{}, S0{}, No{}, blk, Xb, Xa);
        step(S2{}, S0{}, No{}, blk, Xa, Xb);
        step(S3{}, S0{}, No{}, blk, Xb, Xa);
        step(S0{}, S1{}, No{}, blk + 1, Xa, Xb);
        step(S1{}, S1{}, No{}, blk + 1, Xb, Xa);
        step(S2{}, S1{}, No{}, blk + 1, Xa, Xb);
        step(S3{}, S1{}, No{}, blk + 1, Xb, Xa);
    }
    if (blk < blocks) {
        step(S0{}, S0{}, Yes{}, blk, Xa, Xb);
        step(S1{}, S0{}, Yes{}, blk, Xb, Xa);
        step(S2{}, S0{}, Yes{}, blk, Xa, Xb);
        step(S3{}, S0{}, Yes{}, blk, Xb, Xa);
    }
    MOSS_WAIT_VM(0);  // every copy has landed before the workgroup's LDS is released
    if constexpr (SILU) {
        // once every wave's copies have landed (each waited for its own above; the barrier makes
        // that all of them) no wave reads or writes the activation buffers.  Each wave pair hands
        // half of its bf16 results to the other through them -- the gate waves token tiles 2, 3,
        // the up waves tiles 0, 1 -- so that all four waves evaluate the SiLU: wave w & 1 of a
        // pair owns rows 32 (w & 1) .. + 31, the gate waves finish tiles 0, 1, the up waves 2, 3.
        // Slot: pairs of consecutive elements of one lane per 32-bit word.
        __syncthreads();
        uint32_t* xu = reinterpret_cast<uint32_t*>(Xa);  // [from up | from gate] x 2 x 2 tiles x 8 x 64
        const bool up = wave >= 2;
        const int rw = wave & 1;
        auto slot = [&](int from_up, int jj, int pr) { return (((from_up * 2 + rw) * 2 + jj) * 8 + pr) * 64 + lane; };
#pragma unroll
        for (int jj = 0; jj < 2; ++jj)
#pragma unroll
            for (int e = 0; e < 16; e += 2) {
                const int j = up ? jj : jj + 2;  // the tiles the other pair finishes
                xu[slot(up, jj, e / 2)] = pack_bf16x2(acc[j][e], acc[j][e + 1]);
            }
        __syncthreads();
#pragma unroll
        for (int jj = 0; jj < 2; ++jj) {
            const int j = up ? jj + 2 : jj;
            const int m = m0 + 32 * j + (lane & 31);
            if (m >= M) continue;
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const int n = n0 + 32 * rw + 8 * q + 4 * (lane >> 5);
                if (n >= N) continue;  // N % 4 == 0: the quad is all in range or all out
                // the other pair's values for this tile: it stored its tile j - 2 (up) / j (gate)
                // at index jj
                const uint32_t o01 = xu[slot(!up, jj, 2 * q)], o23 = xu[slot(!up, jj, 2 * q + 1)];
                const float m0v = round_bf16(acc[j][4 * q]), m1v = round_bf16(acc[j][4 * q + 1]);
                const float m2v = round_bf16(acc[j][4 * q + 2]), m3v = round_bf16(acc[j][4 * q + 3]);
                const float x0 = bf16_lo(o01), x1 = bf16_hi(o01), x2 = bf16_lo(o23), x3 = bf16_hi(o23);
                uint2 o;
                if (up) {  // own values are up, the others gate
                    o.x = pack_bf16x2(silu_mul_bf16(x0, m0v), silu_mul_bf16(x1, m1v));
                    o.y = pack_bf16x2(silu_mul_bf16(x2, m2v), silu_mul_bf16(x3, m3v));
                } else {
                    o.x = pack_bf16x2(silu_mul_bf16(m0v, x0), silu_mul_bf16(m1v, x1));
                    o.y = pack_bf16x2(silu_mul_bf16(m2v, x2), silu_mul_bf16(m3v, x3));
                }
                *reinterpret_cast<uint2*>(Y + (size_t)m * N + n) = o;
            }
        }
        return;
    }
    if constexpr (QKR) {
        // The tile is one head of 128 tokens.  Its bf16 products (rounded as the plain store rounds
        // them) are staged token-major in the activation buffers -- rows 0..63 in Xa, 64..127 in
        // Xb, 8-byte chunk c of row r at c ^ (r & 31), so the 32 rows of one store hit distinct
        // banks -- then each token row goes through head4_norm_rope on 16 lanes, 16 rows per pass.
        constexpr int QH = 32, KH = 8, D = 128;
        const int head = n0 / D, jl = tid & 15;
        auto ld4 = [](const uint16_t* p) { return *reinterpret_cast<const uint2*>(p); };
        // this thread's 8 token rows r = 16 pass + tid / 16: positions first, then (for query and key
        // heads) the weights and all cos / sin quads, so their latencies overlap the staging
        int64_t pos[8];
#pragma unroll
        for (int pass = 0; pass < 8; ++pass) {
            const int m = min(m0 + 16 * pass + (tid >> 4), M - 1);
            pos[pass] = min(max(qr.positions[m], (int64_t)0), (int64_t)(qr.L - 1));
        }
        auto chunk = [&](int r, int c) {
            return reinterpret_cast<uint2*>((r < 64 ? Xa : Xb) + (r & 63) * 128 + 4 * (c ^ (r & 31)));
        };
        __syncthreads();  // every wave's copies have landed; no wave reads the buffers any more
#pragma unroll
        for (int j = 0; j < JT; ++j)
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                uint2 o;
                o.x = pack_bf16x2(acc[j][4 * q], acc[j][4 * q + 1]);
                o.y = pack_bf16x2(acc[j][4 * q + 2], acc[j][4 * q + 3]);
                *chunk(32 * j + (lane & 31), 8 * wave + 2 * q + (lane >> 5)) = o;
            }
        if (head >= QH + KH) {  // value heads: the rounded products as they are
            __syncthreads();
#pragma unroll
            for (int pass = 0; pass < 8; ++pass) {
                const int r = 16 * pass + (tid >> 4);
                if (m0 + r >= M) continue;
                uint16_t* vd = qr.v_cache + ((size_t)(head - QH - KH) * qr.L + pos[pass]) * D;
                *reinterpret_cast<uint2*>(vd + 4 * jl) = *chunk(r, jl);
                *reinterpret_cast<uint2*>(vd + 64 + 4 * jl) = *chunk(r, 16 + jl);
            }
            return;
        }
        const uint16_t* wt = head < QH ? qr.q_weight : qr.k_weight;
        const uint2 wa = ld4(wt + 4 * jl), wb = ld4(wt + 64 + 4 * jl);
        uint2 cs[8][4];
#pragma unroll
        for (int pass = 0; pass < 8; ++pass) {
            const uint16_t* cr = qr.cos_t + (size_t)pos[pass] * D;
            const uint16_t* sr = qr.sin_t + (size_t)pos[pass] * D;
            cs[pass][0] = ld4(cr + 4 * jl);
            cs[pass][1] = ld4(cr + 64 + 4 * jl);
            cs[pass][2] = ld4(sr + 4 * jl);
            cs[pass][3] = ld4(sr + 64 + 4 * jl);
        }
        __syncthreads();
        // each token row through head4_norm_rope on 16 lanes, 16 rows per pass
#pragma unroll
        for (int pass = 0; pass < 8; ++pass) {
            const int r = 16 * pass + (tid >> 4), m = m0 + r;
            if (m >= M) continue;  // whole 16-lane groups
            uint2 lo, hi;
            head4_norm_rope(*chunk(r, jl), *chunk(r, 16 + jl), wa, wb, cs[pass][0], cs[pass][1], cs[pass][2],
                            cs[pass][3], qr.eps, lo, hi);
            uint16_t* dst = head < QH ? Y + ((size_t)m * QH + head) * D
                                      : qr.k_cache + ((size_t)(head - QH) * qr.L + pos[pass]) * D;
            *reinterpret_cast<uint2*>(dst + 4 * jl) = lo;
            *reinterpret_cast<uint2*>(dst + 64 + 4 * jl) = hi;
        }
        return;
    }
    // C[n][m] of the 32 x 32 tile (n0 + 32 wave, m0 + 32 j): as in w4g32_gemm_t_kernel
#pragma unroll
    for (int j = 0; j < JT; ++j) {
        const int m = m0 + 32 * j + (lane & 31);
        if (m >= M) continue;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const int n = n0 + 32 * wave + 8 * q + 4 * (lane >> 5);
            if (n >= N) continue;
            const float v0 = acc[j][4 * q], v1 = acc[j][4 * q + 1], v2 = acc[j][4 * q + 2], v3 = acc[j][4 * q + 3];
            if constexpr (SPLIT) {
                *reinterpret_cast<float4*>(part + ((size_t)blockIdx.y * M + m) * N + n) = make_float4(v0, v1, v2, v3);
            } else {
                uint2 o;
                o.x = pack_bf16x2(v0, v1);
                o.y = pack_bf16x2(v2, v3);
                *reinterpret_cast<uint2*>(Y + (size_t)m * N + n) = o;
            }
        }
    }
}

// y[m, n] = bf16(scale[n] * sum_z part[z, m, n]), z ascending; 4 outputs per thread (N % 4 == 0).
__global__ __launch_bounds__(256) void gemm_reduce(const float* __restrict__ part, const float* __restrict__ row_scale,
                                                   uint16_t* __restrict__ Y, int MN, int N, int S) {
    const int i = 4 * (blockIdx.x * blockDim.x + threadIdx.x);
    if (i >= MN) return;
    float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
    for (int z = 0; z < S; ++z) {
        const float4 v = *reinterpret_cast<const float4*>(part + (size_t)z * MN + i);
        acc.x += v.x;
        acc.y += v.y;
        acc.z += v.z;
        acc.w += v.w;
    }
    const int n = i % N;  // the 4 outputs share a row
    float4 s = make_float4(1.f, 1.f, 1.f, 1.f);
    if (row_scale) s = make_float4(row_scale[n], row_scale[n + 1], row_scale[n + 2], row_scale[n + 3]);
    uint2 o;
    o.x = pack_bf16x2(acc.x * s.x, acc.y * s.y);
    o.y = pack_bf16x2(acc.z * s.z, acc.w * s.w);
    *reinterpret_cast<uint2*>(Y + i) = o;
}

// ---------------------------------------------------------------------------------------------
// Small M (up to 32 tokens INT4, 16 e4m3; 2 to 4 INT4 tokens mostly take the multi-token GEMV,
// see launch_gemm): weight streaming.  A workgroup owns 16 weight rows over
// the whole of K, so every weight byte is read once per call and no partial sums leave the
// workgroup; ceil(N / 16) workgroups of 8 waves, wave w taking the w-th eighth of K, 4 groups of
// 32 inputs (a quad) per step.  One v_mfma_f32_16x16x32_bf16 per group and token tile: lane
// (j, q) = (lane % 16, lane / 16) holds inputs 32 g + 8 q .. + 7 of group g, as the A operand 8
// weights of row n0 + j (one word of INT4 codes dequantized bit-exactly in registers, or 8 e4m3
// bytes) and as the B operand the same 8 inputs of token 16 tt + j, loaded straight from global
// memory (the activations, at most 32 x K bf16, stay in L2; the 4 lanes of a token read 64
// contiguous bytes).  The weights are loaded a whole group per lane (lane (j, q) takes group
// g + q of the quad, 16 bytes INT4 / 32 bytes e4m3) and then transposed across the 4 lane rows
// with v_permlane32_swap / v_permlane16_swap, so that lane (j, q) holds word q of each of the
// quad's groups.  The 8 waves' 16 x 16 fp32 tiles are added in LDS in wave order
// (deterministic), then scaled (FP8 row scale) and rounded to bf16.  Tokens beyond M load row
// M - 1 and are not stored.  INT4 scales and zero points come 8 groups per load (16 and 8 bytes).
constexpr int kStreamRows = 16;
constexpr int kStreamWaves = 8;

// 4 x 4 transpose across the four 16-lane rows: afterwards register t of row q holds what
// register q of row t held.
__device__ __forceinline__ void rows_transpose(uint32_t& r0, uint32_t& r1, uint32_t& r2, uint32_t& r3) {
    auto a = __builtin_amdgcn_permlane32_swap(r0, r2, false, false);
    auto b = __builtin_amdgcn_permlane32_swap(r1, r3, false, false);
    auto c = __builtin_amdgcn_permlane16_swap(a[0], b[0], false, false);
    auto d = __builtin_amdgcn_permlane16_swap(a[1], b[1], false, false);
    r0 = c[0];
    r1 = c[1];
    r2 = d[0];
    r3 = d[1];
}

template <int FMT, int TT>
__global__ __launch_bounds__(512) void stream_gemm_kernel(const uint16_t* __restrict__ X, const uint8_t* __restrict__ W,
                                                          const uint16_t* __restrict__ sc,
                                                          const uint8_t* __restrict__ zp,
                                                          const float* __restrict__ row_scale,
                                                          uint16_t* __restrict__ Y, int M, int N, int K) {
    constexpr int DQ = 4;                                // quads whose loads are in flight
    constexpr int CW = FMT == kInt4G32 ? 4 : 8;          // weight words per lane per quad
    __shared__ float4 red[kStreamWaves][TT][64];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int n0 = blockIdx.x * kStreamRows, q = lane >> 4, j = lane & 15;
    const int G = K >> 5, S = G / kStreamWaves;  // groups per wave (a multiple of 16)
    const int gw = wave * S;                      // the wave's first group
    const size_t row = (size_t)min(n0 + j, N - 1);
    const uint16_t* xr[TT];
#pragma unroll
    for (int tt = 0; tt < TT; ++tt) xr[tt] = X + (size_t)min(16 * tt + j, M - 1) * K + 32 * gw + 8 * q;

    // quad d: groups gw + 4 d .. + 3
    auto load_x = [&](u32x4_t (&xv)[4][TT], int d) {
#pragma unroll
        for (int t = 0; t < 4; ++t)
#pragma unroll
            for (int tt = 0; tt < TT; ++tt) xv[t][tt] = *reinterpret_cast<const u32x4_t*>(xr[tt] + 32 * (4 * d + t));
    };
    auto load_w = [&](uint32_t (&w)[CW], int d) {
        const int g = gw + 4 * d + q;
        if constexpr (FMT == kInt4G32) {
            const uint4 v = reinterpret_cast<const uint4*>(W)[row * G + g];
            w[0] = v.x; w[1] = v.y; w[2] = v.z; w[3] = v.w;
        } else {
            const uint4* src = reinterpret_cast<const uint4*>(W + row * K + 32 * g);
            const uint4 v0 = src[0], v1 = src[1];
            w[0] = v0.x; w[1] = v0.y; w[2] = v0.z; w[3] = v0.w;
            w[4] = v1.x; w[5] = v1.y; w[6] = v1.z; w[7] = v1.w;
        }
    };
    // INT4: scales (8 bf16) and zero bytes (8, one nibble side) of groups gw + 8 b .. + 7
    auto load_sz = [&](uint4& sv, uint2& zv, uint32_t& zsh, int b) {
        const int g = gw + 8 * b;
        int zb;
        zero_loc(g, G, zb, zsh);
        sv = *reinterpret_cast<const uint4*>(sc + row * G + g);
        zv = *reinterpret_cast<const uint2*>(zp + row * (G >> 1) + zb);
    };

    f32x4_t acc[TT];
#pragma unroll
    for (int tt = 0; tt < TT; ++tt) acc[tt] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    const int quads = S / 4;
    uint32_t cw[DQ][CW];
    u32x4_t xv[DQ][4][TT];
    uint4 sv[2] = {}, sv_n[2] = {};
    uint2 zv[2] = {}, zv_n[2] = {};
    uint32_t zsh[2] = {}, zsh_n[2] = {};
    if constexpr (FMT == kInt4G32) {
        load_sz(sv[0], zv[0], zsh[0], 0);
        load_sz(sv[1], zv[1], zsh[1], 1);
        if (quads > 4) {
            load_sz(sv_n[0], zv_n[0], zsh_n[0], 2);
            load_sz(sv_n[1], zv_n[1], zsh_n[1], 3);
        }
    }
#pragma unroll
    for (int i = 0; i < DQ; ++i) {
        load_w(cw[i], i);  // quads >= 4 >= DQ
        load_x(xv[i], i);
    }
    const MixedUnpack mu = make_mixed_unpack();
    for (int d0 = 0; d0 < quads; d0 += 4) {  // quads % 4 == 0; DQ divides 4
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const int d = d0 + u, i = u % DQ;
            pin();
            // lane (j, q): word q of each group of the quad (INT4), words 2 q, 2 q + 1 (e4m3)
            uint32_t wq[CW];
#pragma unroll
            for (int c = 0; c < CW; ++c) wq[c] = cw[i][c];
            if constexpr (FMT == kInt4G32) {
                rows_transpose(wq[0], wq[1], wq[2], wq[3]);
            } else {
                // words 2 t, 2 t + 1 of group g + q hold inputs 8 t .. 8 t + 7
                rows_transpose(wq[0], wq[2], wq[4], wq[6]);
                rows_transpose(wq[1], wq[3], wq[5], wq[7]);
            }
            // the weight slot is free: quad d + DQ into it (a wave-uniform branch: no refill past
            // the wave's last quad)
            if (d + DQ < quads) load_w(cw[i], d + DQ);
            pin();
#pragma unroll
            for (int t = 0; t < 4; ++t) {  // group gw + 4 d + t
                uint32_t a[4];
                if constexpr (FMT == kInt4G32) {
                    const int gi = 4 * (u & 1) + t;  // within the 8-group scale block u / 2
                    const uint4& s8 = sv[u >> 1];
                    const uint32_t sw = gi < 2 ? s8.x : gi < 4 ? s8.y : gi < 6 ? s8.z : s8.w;
                    const uint32_t zq = ((gi < 4 ? zv[u >> 1].x : zv[u >> 1].y) >> (8 * (gi & 3) + zsh[u >> 1])) & 15u;
                    const GroupDequant gd = group_dequant(sw >> (16 * (gi & 1)), zq);
                    dequant_word_mixed(wq[t], mu, gd.s_lo, gd.s_hi, gd.s, gd.bias_bf16, gd.bias_f16, a);
                } else {
                    a[0] = fp8x2_to_bf16x2<false>(wq[2 * t]);
                    a[1] = fp8x2_to_bf16x2<true>(wq[2 * t]);
                    a[2] = fp8x2_to_bf16x2<false>(wq[2 * t + 1]);
                    a[3] = fp8x2_to_bf16x2<true>(wq[2 * t + 1]);
                }
                const bf16x8_t av = __builtin_bit_cast(bf16x8_t, u32x4_t{a[0], a[1], a[2], a[3]});
#pragma unroll
                for (int tt = 0; tt < TT; ++tt)
                    acc[tt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(av, __builtin_bit_cast(bf16x8_t, xv[i][t][tt]),
                                                                      acc[tt], 0, 0, 0);
            }
            pin();
            if (d + DQ < quads) load_x(xv[i], d + DQ);  // the activation slot, once the MFMAs have read it
            if (FMT == kInt4G32 && u == 3) {            // the next 16 groups' scale blocks
                sv[0] = sv_n[0]; zv[0] = zv_n[0]; zsh[0] = zsh_n[0];
                sv[1] = sv_n[1]; zv[1] = zv_n[1]; zsh[1] = zsh_n[1];
                if (d0 + 8 < quads) {
                    load_sz(sv_n[0], zv_n[0], zsh_n[0], d0 / 2 + 4);
                    load_sz(sv_n[1], zv_n[1], zsh_n[1], d0 / 2 + 5);
                }
            }
        }
    }
    // D[r][c] of the 16 x 16 tile: lane l, element e -> weight row 4 (l / 16) + e, token l % 16
#pragma unroll
    for (int tt = 0; tt < TT; ++tt) red[wave][tt][lane] = make_float4(acc[tt][0], acc[tt][1], acc[tt][2], acc[tt][3]);
    __syncthreads();
    if (tid >= TT * 64) return;
    const int tt = tid >> 6, l = tid & 63;
    float4 sum = red[0][tt][l];
#pragma unroll
    for (int w = 1; w < kStreamWaves; ++w) {
        const float4 r = red[w][tt][l];
        sum.x += r.x;
        sum.y += r.y;
        sum.z += r.z;
        sum.w += r.w;
    }
    float v[4] = {sum.x, sum.y, sum.z, sum.w};
    const int n = n0 + 4 * (l >> 4), m = 16 * tt + (l & 15);
    if (m >= M || n >= N) return;  // N % 4 == 0: the 4 rows are all in range or all out
    if (FMT == kFp8E4M3 && row_scale) {
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] *= row_scale[n + e];
    }
    *reinterpret_cast<uint2*>(Y + (size_t)m * N + n) = make_uint2(pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3]));
}

// Shapes and pointers the streaming kernel takes: 8 waves x 4 steps of 4 groups of K (INT4: the
// 8 zero bytes of a scale block on one nibble side), 4-row output stores, 16-byte weight,
// activation and scale loads, 8-byte zero-point loads; and at least 128 workgroups.
bool stream_shape(int FMT, int M, int K, int N, const void* x, const void* qw, const void* sc, const void* zp,
                  const void* y) {
    // up to 32 tokens for INT4 and 16 for e4m3 it is faster on MI355X than the tiles (measured at
    // K = N = 4096: INT4 M = 32 11.9 vs 12.8 us, M = 64 18.8 vs 16.9 us; e4m3 M = 64 19.8 vs 13.3 us):
    // every workgroup reads all M x K activations, which outweighs the weight stream as M grows
    if (M < 1 || M > (FMT == kInt4G32 ? 32 : 16) || N % 4 || N < 128 * kStreamRows) return false;
    if (!(MOSS_ALIGNED(x, 16) && MOSS_ALIGNED(qw, 16) && MOSS_ALIGNED(y, 8))) return false;
    if (K % 4096) return false;  // K / 256 groups per wave: whole 4-quad steps
    return FMT == kFp8E4M3 || (MOSS_ALIGNED(sc, 16) && MOSS_ALIGNED(zp, 8));
}

template <int FMT>
void launch_stream(const void* x, const void* qw, const void* sc, const void* zp, const float* row_scale, void* y,
                   int M, int K, int N, hipStream_t st) {
    const dim3 grid((unsigned)((N + kStreamRows - 1) / kStreamRows));
#define MOSS_STREAM(TTV)                                                                                         \
    hipLaunchKernelGGL((stream_gemm_kernel<FMT, TTV>), grid, dim3(64 * kStreamWaves), 0, st, (const uint16_t*)x, \
                       (const uint8_t*)qw, (const uint16_t*)sc, (const uint8_t*)zp, row_scale, (uint16_t*)y, M, N, K)
    if (M <= 16) MOSS_STREAM(1);
    else MOSS_STREAM(2);  // M <= 32 (stream_shape)
#undef MOSS_STREAM
}

struct Plan {
    int bm, bn, split;
    bool reg;  // the register-weight 128 x 128 INT4 tile
};

// Shapes the register-weight tile takes: whole blocks of kTs steps, 4-output stores, and for
// INT4 the 8 zero bytes of every block on one nibble side of their 128-group chunk (the last
// chunk a multiple of 16 groups long) and 16-byte scale rows.
bool reg_tile_shape(int K, int N, bool int4) {
    const int G = K / 32;
    return int4 && N % 4 == 0 && (K / kBK) % kTs == 0 && G % 16 == 0 && (G % 128) % 16 == 0;
}

// INT4: the register-weight tile, 32, 64 or 128 tokens deep.  M > 64 (MFMA-bound): split K (2..8,
// >= 2 blocks each) while the doubled workgroup count still fits one per CU.  M <= 64 (bound by
// the weight stream): split while the workgroups fit two per CU and the fp32 partials (written
// and read back once) stay below half the weight bytes.  Shapes it does not take use the LDS
// tiles: 64-row tiles for M <= 64; 128-wide N tiles when they already give >= 256 workgroups; a
// K split (2..8) for M <= 256 while the tiles give fewer than 256 workgroups, and a split of 2
// up to M = 1024 when the tiles give at most 256 (the fp32 partials cost 8 M N bytes per split).
Plan plan_lds(int M, int K, int N);

Plan plan_gemm(int M, int K, int N, bool int4) {
    if (!reg_tile_shape(K, N, int4)) return plan_lds(M, K, N);
    Plan p;
    p.reg = true;
    {
        p.bm = M <= 32 ? 32 : M <= 64 ? 64 : 128;
        p.bn = 128;
        p.split = 1;
        const long tiles = (long)((M + p.bm - 1) / p.bm) * ((N + 127) / 128);
        const int steps = K / kBK;
        const double wbytes = (double)N * K * 0.5625;  // codes, scales, zero points
        // M > 64 (the LDS-copy tile, three workgroups per CU): split only up to one workgroup per
        // CU; measured over M = 128 .. 2048, a deeper split costs more in partial sums and their
        // reduction than the extra workgroups gain
        const long cap = M <= 64 ? 512 : 256;
        while (p.split < 16 && tiles * p.split * 2 <= cap && steps % (2 * p.split * kTs) == 0 &&
               (M <= 64 ? 2.0 * p.split * M * N * 4 <= 0.5 * wbytes
                        : (p.split < 8 && steps / (2 * p.split) >= 2 * kTs)))
            p.split *= 2;
        return p;
    }
}

Plan plan_lds(int M, int K, int N) {
    Plan p;
    p.reg = false;
    p.bm = M <= 64 ? 64 : 128;
    const long mt = (M + p.bm - 1) / p.bm;
    p.bn = mt * ((N + 127) / 128) >= 256 ? 128 : 64;
    const long tiles = mt * ((N + p.bn - 1) / p.bn);
    const int steps = K / kBK;
    p.split = 1;
    if (N % 4 == 0 && M <= 256) {
        while (p.split < 8 && tiles * p.split < 256 && steps % (2 * p.split) == 0 && steps / (2 * p.split) >= 4)
            p.split *= 2;
    } else if (N % 4 == 0 && M <= 1024 && tiles <= 256 && steps % 4 == 0 && steps / 4 >= 4) {
        p.split = 2;  // one workgroup per CU would leave half of each CU's wave slots empty
    }
    return p;
}

template <int BM, int BN, int FMT, bool TAIL>
void launch_tile2(const Plan& p, const void* x, const void* qw, const void* sc, const void* zp, void* y, void* part,
                  int M, int K, int N, const float* row_scale, hipStream_t st) {
    const dim3 grid((unsigned)(((M + BM - 1) / BM) * ((N + BN - 1) / BN)), (unsigned)p.split);
    if (p.split > 1)
        hipLaunchKernelGGL((w4g32_gemm_kernel<BM, BN, FMT, true, TAIL>), grid, dim3(256), 0, st, (const uint16_t*)x,
                           (const uint4*)qw, (const uint16_t*)sc, (const uint8_t*)zp, (uint16_t*)y, (float*)part, M,
                           N, K, row_scale);
    else
        hipLaunchKernelGGL((w4g32_gemm_kernel<BM, BN, FMT, false, TAIL>), grid, dim3(256), 0, st, (const uint16_t*)x,
                           (const uint4*)qw, (const uint16_t*)sc, (const uint8_t*)zp, (uint16_t*)y, (float*)part, M,
                           N, K, row_scale);
}

template <int BM, int BN, int FMT>
void launch_tile(const Plan& p, const void* x, const void* qw, const void* sc, const void* zp, void* y, void* part,
                 int M, int K, int N, const float* row_scale, hipStream_t st) {
    if ((K / kBK / p.split) % stages_for<BM, BN>() == 0)
        launch_tile2<BM, BN, FMT, false>(p, x, qw, sc, zp, y, part, M, K, N, row_scale, st);
    else
        launch_tile2<BM, BN, FMT, true>(p, x, qw, sc, zp, y, part, M, K, N, row_scale, st);
}

template <int JT>
void launch_reg(const Plan& p, const void* x, const void* qw, const void* sc, const void* zp, void* y, void* ws,
                int M, int K, int N, hipStream_t st) {
    const dim3 grid((unsigned)(((M + 32 * JT - 1) / (32 * JT)) * ((N + 127) / 128)), (unsigned)p.split);
    if constexpr (JT == 4) {
        if (p.split > 1)
            hipLaunchKernelGGL((w4g32_gemm_tdma_kernel<true>), grid, dim3(256), 0, st, (const uint16_t*)x,
                               (const uint4*)qw, (const uint16_t*)sc, (const uint8_t*)zp, (uint16_t*)y, (float*)ws, M, N, K,
                               QkRope{});
        else
            hipLaunchKernelGGL((w4g32_gemm_tdma_kernel<false>), grid, dim3(256), 0, st, (const uint16_t*)x,
                               (const uint4*)qw, (const uint16_t*)sc, (const uint8_t*)zp, (uint16_t*)y, (float*)ws, M, N, K,
                               QkRope{});
        return;
    }
    if (p.split > 1)
        hipLaunchKernelGGL((w4g32_gemm_t_kernel<JT, true>), grid, dim3(256), 0, st, (const uint16_t*)x,
                           (const uint4*)qw, (const uint16_t*)sc, (const uint8_t*)zp, (uint16_t*)y, (float*)ws, M, N, K);
    else
        hipLaunchKernelGGL((w4g32_gemm_t_kernel<JT, false>), grid, dim3(256), 0, st, (const uint16_t*)x,
                           (const uint4*)qw, (const uint16_t*)sc, (const uint8_t*)zp, (uint16_t*)y, (float*)ws, M, N, K);
}

// split_out: when non-null, a K-split plan leaves its fp32 partials in ws for the caller to reduce
// (no gemm_reduce launch) and *split_out receives the split (1: y holds the product).
template <int FMT>
int launch_gemm(const void* x, const void* qw, const void* sc, const void* zp, void* y, int M, int K, int N,
                const float* row_scale, void* ws, long long ws_bytes, hipStream_t st, int* split_out = nullptr) {
    if (split_out) *split_out = 1;
    // INT4, 2 to 4 tokens: the exact GEMV holding every token's x in registers reads the weights
    // once, on the VALU, each row of y equal to the single-token GEMV of its token.  Faster than the
    // weight-streaming kernel (measured on MI355X, 2 / 3 / 4 tokens: K = 4096, N = 12288: 9.8 /
    // 11.6 / 13.7 against 14.6 / 15.1 / 15.6 us; N = 24576: 16.5 / 20.6 / 24.0 against 27.4 / 28.2
    // / 29.3 us; K = 12288, N = 4096: 9.9 / 13.1 against 13.0 / 13.3 us) except 4 tokens at
    // K > 4096 (15.2 against 13.7 us), which stays on the streaming kernel.
    if (FMT == kInt4G32 && w4g32_gemv_tokens_shape(M, K) && (M <= 3 || K <= 4096) && MOSS_ALIGNED(x, 16) &&
        MOSS_ALIGNED(qw, 16))
        return w4g32_gemv_tokens_launch(x, qw, sc, zp, y, M, K, N, st);
    if (stream_shape(FMT, M, K, N, x, qw, sc, zp, y)) {
        launch_stream<FMT>(x, qw, sc, zp, row_scale, y, M, K, N, st);
        return moss_launch_status();
    }
    Plan p = plan_gemm(M, K, N, FMT == kInt4G32);
    // the register-weight tile stores 4 outputs (8 bytes) at a time and loads scales and zero
    // bytes 16 and 8 at a time
    if (p.reg && !(MOSS_ALIGNED(y, 8) && MOSS_ALIGNED(sc, 16) && MOSS_ALIGNED(zp, 8)))
        p = plan_lds(M, K, N);
    if (p.split > 1 &&
        (!ws || ws_bytes < (long long)p.split * M * N * 4 || !MOSS_ALIGNED(ws, 16) || !MOSS_ALIGNED(y, 8)))
        p.split = 1;
    if (p.reg) {
        if (p.bm == 32) launch_reg<1>(p, x, qw, sc, zp, y, ws, M, K, N, st);
        else if (p.bm == 64) launch_reg<2>(p, x, qw, sc, zp, y, ws, M, K, N, st);
        else launch_reg<4>(p, x, qw, sc, zp, y, ws, M, K, N, st);
    } else if (p.bm == 64 && p.bn == 64) launch_tile<64, 64, FMT>(p, x, qw, sc, zp, y, ws, M, K, N, row_scale, st);
    else if (p.bm == 64) launch_tile<64, 128, FMT>(p, x, qw, sc, zp, y, ws, M, K, N, row_scale, st);
    else if (p.bn == 64) launch_tile<128, 64, FMT>(p, x, qw, sc, zp, y, ws, M, K, N, row_scale, st);
    else launch_tile<128, 128, FMT>(p, x, qw, sc, zp, y, ws, M, K, N, row_scale, st);
    if (p.split > 1 && split_out) {
        *split_out = p.split;
    } else if (p.split > 1) {
        const int mn = M * N;
        hipLaunchKernelGGL(gemm_reduce, dim3((unsigned)((mn / 4 + 255) / 256)), dim3(256), 0, st, (const float*)ws,
                           FMT == kFp8E4M3 ? row_scale : nullptr, (uint16_t*)y, mn, N, p.split);
    }
    return moss_launch_status();
}

}  // namespace

// FP8 e4m3 rows [N, K] with optional fp32 row scales; arguments checked by the caller.
int fp8_gemm_launch(const void* x, const void* w, const float* row_scale, void* y, int M, int K, int N, void* ws,
                    long long ws_bytes, hipStream_t stream) {
    return launch_gemm<kFp8E4M3>(x, w, nullptr, nullptr, y, M, K, N, row_scale, ws, ws_bytes, stream);
}

// The gate||up GEMM with the SiLU*mul epilogue runs fused where moss_w4g32_gemm would run the
// 128-token copy tile unsplit on all 2 N rows (so the two agree bit for bit): M > 64, the register
// tile's shapes, no K split in the plan, and the tile's pointer alignment.
bool silu_fusable_shape(int M, int K, int N) {
    if (M <= 64 || N % 4) return false;
    const Plan p = plan_gemm(M, K, 2 * N, true);
    return p.reg && p.bm == 128 && p.split == 1;
}

long long align16(long long b) { return (b + 15) & ~15ll; }

// The QKV projection (N = 6144) with the q/k-norm + RoPE epilogue: fused under the same conditions.
constexpr int kQkvN = 6144;
bool qk_rope_fusable_shape(int M, int K) {
    if (M <= 64) return false;
    const Plan p = plan_gemm(M, K, kQkvN, true);
    return p.reg && p.bm == 128 && p.split == 1;
}

// One workspace serves both formats and the LDS-tile fallback: the largest plan's partial sums.
long long gemm_workspace_bytes(int M, int K, int N) {
    long long bytes = 0;
    for (const Plan& p : {plan_gemm(M, K, N, true), plan_gemm(M, K, N, false), plan_lds(M, K, N)})
        if (p.split > 1) bytes = std::max(bytes, (long long)p.split * M * N * 4);
    return bytes;
}

}  // namespace moss

using namespace moss;

extern "C" int moss_silu_mul(const void* x, void* y, int rows, int n, void* stream);

MOSS_API long long moss_gemm_workspace_bytes(int M, int K, int N) {
    if (M <= 0 || K <= 0 || N <= 0 || K % 64) return 0;
    return gemm_workspace_bytes(M, K, N);
}

MOSS_API int moss_w4g32_gemm(const void* x, const void* qw, const void* sc, const void* zp, void* y, int M, int K,
                             int N, void* workspace, long long workspace_bytes, void* stream) {
    MOSS_CHECK_ARG(x && qw && sc && zp && y && M > 0 && N > 0 && K > 0 && K % 64 == 0);
    MOSS_CHECK_ARG(MOSS_ALIGNED(x, 16) && MOSS_ALIGNED(qw, 16) && workspace_bytes >= 0);
    return launch_gemm<kInt4G32>(x, qw, sc, zp, y, M, K, N, nullptr, workspace, workspace_bytes,
                                 (hipStream_t)stream);
}

// The unfused form keeps the [M, 2 N] gate||up product in the workspace, followed by the GEMM's own
// K-split partials.  The fused tile needs none, but it depends on the alignment of sc, zp and y,
// which the size query does not see: the query returns the unfused form's size for every shape, so
// a workspace of that size always suffices.
MOSS_API long long moss_gemm_silu_workspace_bytes(int M, int K, int N) {
    if (M <= 0 || K <= 0 || N <= 0 || K % 64 || N % 4) return 0;
    return align16((long long)M * 2 * N * 2) + gemm_workspace_bytes(M, K, 2 * N);
}

MOSS_API int moss_w4g32_gemm_silu(const void* x, const void* qw, const void* sc, const void* zp, void* y, int M, int K,
                                  int N, void* workspace, long long workspace_bytes, void* stream) {
    MOSS_CHECK_ARG(x && qw && sc && zp && y && M > 0 && N > 0 && K > 0 && K % 64 == 0 && N % 4 == 0);
    MOSS_CHECK_ARG(MOSS_ALIGNED(x, 16) && MOSS_ALIGNED(qw, 16) && workspace_bytes >= 0);
    hipStream_t st = (hipStream_t)stream;
    if (silu_fusable_shape(M, K, N) && MOSS_ALIGNED(y, 8) && MOSS_ALIGNED(sc, 16) && MOSS_ALIGNED(zp, 8)) {
        const dim3 grid((unsigned)(((M + 127) / 128) * ((N + 63) / 64)));
        hipLaunchKernelGGL((w4g32_gemm_tdma_kernel<false, true>), grid, dim3(256), 0, st, (const uint16_t*)x,
                           (const uint4*)qw, (const uint16_t*)sc, (const uint8_t*)zp, (uint16_t*)y, (float*)nullptr,
                           M, N, K, QkRope{});
        return moss_launch_status();
    }
    const long long inter = align16((long long)M * 2 * N * 2);
    MOSS_CHECK_ARG(workspace && MOSS_ALIGNED(workspace, 16) && workspace_bytes >= inter);
    char* ws = (char*)workspace;
    if (int rc = launch_gemm<kInt4G32>(x, qw, sc, zp, ws, M, K, 2 * N, nullptr, ws + inter, workspace_bytes - inter, st))
        return rc;
    return moss_silu_mul(ws, y, M, N, stream);
}

extern "C" int moss_rmsnorm(const void* x, const void* res, const void* w, void* sum_out, void* y, int rows, int n,
                            float eps, void* stream);
extern "C" int moss_qk_norm_rope_kv(const void* qkv, const void* q_weight, const void* k_weight, const void* cos,
                                    const void* sin, void* q_out, void* k_cache, void* v_cache, const void* positions,
                                    int L, int ntok, float eps, int cos_by_position, void* stream);

// The unfused form keeps the [M, 6144] QKV product in the workspace, followed by the GEMM's own
// K-split partials; returned for every shape, as for moss_gemm_silu_workspace_bytes.
MOSS_API long long moss_gemm_qk_rope_workspace_bytes(int M, int K) {
    if (M <= 0 || K <= 0 || K % 64) return 0;
    return align16((long long)M * kQkvN * 2) + gemm_workspace_bytes(M, K, kQkvN);
}

MOSS_API int moss_w4g32_gemm_qk_rope(const void* x, const void* qw, const void* sc, const void* zp,
                                     const void* q_weight, const void* k_weight, const void* cos, const void* sin,
                                     void* q_out, void* k_cache, void* v_cache, const void* positions, int M, int K,
                                     int L, float eps, void* workspace, long long workspace_bytes, void* stream) {
    MOSS_CHECK_ARG(x && qw && sc && zp && q_weight && k_weight && cos && sin && q_out && k_cache && v_cache &&
                   positions && M > 0 && K > 0 && K % 64 == 0 && L > 0 && eps >= 0.f && workspace_bytes >= 0);
    MOSS_CHECK_ARG(MOSS_ALIGNED(x, 16) && MOSS_ALIGNED(qw, 16) && MOSS_ALIGNED(q_weight, 8) &&
                   MOSS_ALIGNED(k_weight, 8) && MOSS_ALIGNED(cos, 8) && MOSS_ALIGNED(sin, 8) &&
                   MOSS_ALIGNED(q_out, 8) && MOSS_ALIGNED(k_cache, 8) && MOSS_ALIGNED(v_cache, 8) &&
                   MOSS_ALIGNED(positions, 8));
    hipStream_t st = (hipStream_t)stream;
    if (qk_rope_fusable_shape(M, K) && MOSS_ALIGNED(sc, 16) && MOSS_ALIGNED(zp, 8)) {
        const QkRope qr{(const uint16_t*)q_weight, (const uint16_t*)k_weight, (const uint16_t*)cos,
                        (const uint16_t*)sin, (uint16_t*)k_cache, (uint16_t*)v_cache, (const int64_t*)positions, L,
                        eps};
        const dim3 grid((unsigned)(((M + 127) / 128) * (kQkvN / 128)));
        hipLaunchKernelGGL((w4g32_gemm_tdma_kernel<false, false, true>), grid, dim3(256), 0, st, (const uint16_t*)x,
                           (const uint4*)qw, (const uint16_t*)sc, (const uint8_t*)zp, (uint16_t*)q_out,
                           (float*)nullptr, M, kQkvN, K, qr);
        return moss_launch_status();
    }
    const long long inter = align16((long long)M * kQkvN * 2);
    MOSS_CHECK_ARG(workspace && MOSS_ALIGNED(workspace, 16) && workspace_bytes >= inter);
    char* ws = (char*)workspace;
    int split = 1;
    if (int rc = launch_gemm<kInt4G32>(x, qw, sc, zp, ws, M, K, kQkvN, nullptr, ws + inter, workspace_bytes - inter,
                                       st, &split))
        return rc;
    if (split > 1)  // the RoPE kernel reduces the partials itself, in split order
        return qk_rope_from_parts((const float*)(ws + inter), split, q_weight, k_weight, cos, sin, q_out, k_cache,
                                  v_cache, positions, L, M, eps, st);
    return moss_qk_norm_rope_kv(ws, q_weight, k_weight, cos, sin, q_out, k_cache, v_cache, positions, L, M, eps, 1,
                                stream);
}

// The O / down projection followed by the residual add and RMSNorm of the prompt pass.  A K-split
// plan's partials go straight into the norm kernel, which reduces them in split order; otherwise
// the product goes to summed_out and the in-place add-RMSNorm kernel runs there (each thread reads
// a chunk before it writes the same chunk).  summed_out and y may not overlap x, residual or each
// other: such calls are refused.
MOSS_API int moss_w4g32_gemm_add_rmsnorm(const void* x, const void* qw, const void* sc, const void* zp,
                                         const void* residual, const void* norm_w, float eps, void* summed_out,
                                         void* y, int M, int K, int N, void* workspace, long long workspace_bytes,
                                         void* stream) {
    MOSS_CHECK_ARG(x && qw && sc && zp && residual && norm_w && summed_out && y && M > 0 && N > 0 && K > 0 &&
                   K % 64 == 0 && N % 8 == 0 && N <= 8192 && eps >= 0.f);
    MOSS_CHECK_ARG(MOSS_ALIGNED(x, 16) && MOSS_ALIGNED(qw, 16) && MOSS_ALIGNED(residual, 16) &&
                   MOSS_ALIGNED(norm_w, 16) && MOSS_ALIGNED(summed_out, 16) && MOSS_ALIGNED(y, 16) &&
                   workspace_bytes >= 0);
    const size_t xb = (size_t)M * K * 2, ob = (size_t)M * N * 2;
    MOSS_CHECK_ARG(!moss_overlaps(summed_out, ob, x, xb) && !moss_overlaps(summed_out, ob, residual, ob) &&
                   !moss_overlaps(y, ob, x, xb) && !moss_overlaps(y, ob, residual, ob) &&
                   !moss_overlaps(y, ob, summed_out, ob));
    hipStream_t st = (hipStream_t)stream;
    int split = 1;
    if (int rc = launch_gemm<kInt4G32>(x, qw, sc, zp, summed_out, M, K, N, nullptr, workspace, workspace_bytes, st,
                                       &split))
        return rc;
    if (split > 1) return addnorm_from_parts((const float*)workspace, split, residual, norm_w, summed_out, y, M, N, eps, st);
    return add_rmsnorm_inplace(summed_out, residual, norm_w, y, M, N, eps, st);
}

// ---------------------------------------------------------------------------------------------
// The allocation-free GEMM: the K-split partial sums go to a file-scope device array instead of a
// caller workspace.  Every plan's partials fit in it (at most 512 workgroups of 128 x 128 fp32
// outputs, 32 MiB).  Each device holds its own copy at its own address, found once per device with
// hipGetSymbolAddress; host code uses only that address, never the array's name.  The partials are
// written in full before the reduction reads them, so nothing needs clearing between calls, but
// calls that overlap on one device share the array and race.
static constexpr long long kScratchBytes = 32ll << 20;
static __device__ __align__(256) float scratch[kScratchBytes / 4];

static constexpr int kMaxScratchDevices = 64;
static void* g_scratch_ptr[kMaxScratchDevices];
static std::mutex g_scratch_mu;

static int scratch_of_current_device(void** out) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return (int)e;
    if (dev < 0 || dev >= kMaxScratchDevices) return (int)hipErrorInvalidDevice;
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_ptr[dev]) {
        void* p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return (int)e;
        if (!p) return (int)hipErrorInvalidSymbol;
        g_scratch_ptr[dev] = p;
    }
    *out = g_scratch_ptr[dev];
    return 0;
}

MOSS_API int moss_w4g32_gemm_noalloc(const void* x, const void* qw, const void* sc, const void* zp, void* y, int M,
                                     int K, int N, void* stream) {
    MOSS_CHECK_ARG(x && qw && sc && zp && y && M > 0 && N > 0 && K > 0 && K % 64 == 0);
    MOSS_CHECK_ARG(MOSS_ALIGNED(x, 16) && MOSS_ALIGNED(qw, 16));
    // a plan whose partials would not fit is refused rather than run differently
    MOSS_CHECK_ARG(gemm_workspace_bytes(M, K, N) <= kScratchBytes);
    void* ws = nullptr;
    if (int rc = scratch_of_current_device(&ws)) return rc;
    return launch_gemm<kInt4G32>(x, qw, sc, zp, y, M, K, N, nullptr, ws, kScratchBytes, (hipStream_t)stream);
}
