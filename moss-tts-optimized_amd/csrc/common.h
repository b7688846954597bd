// Shared device helpers for the gfx950 kernels behind libmoss_hip.so.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#define MOSS_API extern "C" __attribute__((visibility("default")))

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));

// Dequant modes of the decode GEMVs (see include/moss_hip.h).
#define MOSS_DEQUANT_EXACT 0
#define MOSS_DEQUANT_UNROUNDED 1

namespace moss {

constexpr int kWave = 64;

// ---------------------------------------------------------------- bf16 bit helpers
__device__ __forceinline__ float bf16_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }
__device__ __forceinline__ float bf16_bits(uint16_t b) { return __uint_as_float((uint32_t)b << 16); }

// float -> bf16 bits, round to nearest even (one v_cvt_pk_bf16_f32; fp32 denormals are kept,
// NaN stays a quiet NaN).
__device__ __forceinline__ uint16_t f32_to_bf16(float f) { return __builtin_bit_cast(uint16_t, (__bf16)f); }

// Two floats -> a packed bf16 pair (lo in bits 0..15), each rounded to nearest even, in one
// v_cvt_pk_bf16_f32.
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
    const bf16x2_t v = {(__bf16)lo, (__bf16)hi};
    return __builtin_bit_cast(uint32_t, v);
}

// Round a float through bf16 and back (the "x.to(bf16).to(f32)" step).
__device__ __forceinline__ float round_bf16(float f) { return bf16_bits(f32_to_bf16(f)); }

// The SiLU*mul epilogue on bf16 gate and up values: bf16(silu(g)) * u, rounded by the caller
// (src/moss_tts/_runtime/prefill_pointwise.py:18-31).  One definition for every kernel that must
// agree bit for bit.
__device__ __forceinline__ float silu_mul_bf16(float g, float u) { return round_bf16(g / (1.0f + expf(-g))) * u; }

// The same from the fp32 gate and up projection outputs of the decode GEMVs, each rounded to bf16
// first: the bf16 bits of bf16(bf16(silu(bf16(gate))) * bf16(up)) (src/moss_tts/_runtime/dp4a_scaled.py:65-68).
__device__ __forceinline__ uint16_t silu_mul_rounded_bits(float gate, float up) {
    return f32_to_bf16(silu_mul_bf16(round_bf16(gate), round_bf16(up)));
}

// Where group g's zero point sits in a row-packed zp row (blocks of 128 groups: for block c with
// r = min(128, G - 128c) groups, byte 64c + b holds z[128c + b] low and z[128c + r/2 + b] high):
// byte index and bit shift.  Branch-free, so a byte load through it is not followed by a wait at
// the load site; callers that prefetch keep the raw byte and shift until the value is used.
__device__ __forceinline__ void zero_loc(int g, int G, int& byte, uint32_t& shift) {
    const int c0 = g & ~127, r = min(128, G - c0), off = g - c0, hr = r >> 1;
    const int hi = off >= hr;
    byte = (c0 >> 1) + off - hi * hr;
    shift = (uint32_t)hi << 2;
}

__device__ __forceinline__ uint32_t zero_of_group(const uint8_t* __restrict__ zrow, int g, int G) {
    int b;
    uint32_t sh;
    zero_loc(g, G, b, sh);
    return ((uint32_t)zrow[b] >> sh) & 15u;
}

// ---------------------------------------------------------------- cross-lane sums
template <int CTRL>
__device__ __forceinline__ float dpp_move(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xf, 0xf, false));
}

// Sum over the 16 lanes of each DPP row; every lane of the row receives the row sum.
__device__ __forceinline__ float row16_sum(float v) {
    v += dpp_move<0xB1>(v);   // quad_perm [1,0,3,2]
    v += dpp_move<0x4E>(v);   // quad_perm [2,3,0,1]
    v += dpp_move<0x141>(v);  // row_half_mirror: lane i <- lane 7-i within 8
    v += dpp_move<0x140>(v);  // row_mirror: lane i <- lane 15-i within 16
    return v;
}

// Full 64-lane sum, the same value in every lane.  Fixed order, so results are deterministic:
// the 16-lane row sums r0..r3, then (r0 + r1) + (r2 + r3).  v_permlane16_swap(x, x) hands every
// lane the row sums of its own and its neighbouring row (r0 | r1 in rows 0 and 1, r2 | r3 in rows
// 2 and 3) and v_permlane32_swap(x, x) the two halves' results; being commutative, + and max give
// the same bits in every lane, without the readlanes and their SGPR hazards.
__device__ __forceinline__ float wave_sum(float v) {
    v = row16_sum(v);
    const auto p = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    v = __uint_as_float(p[0]) + __uint_as_float(p[1]);
    const auto q = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float(q[0]) + __uint_as_float(q[1]);
}

// Full 64-lane maximum, the same value in every lane (the row maxima combined as in wave_sum).
__device__ __forceinline__ float wave_max(float v) {
    v = fmaxf(v, dpp_move<0xB1>(v));
    v = fmaxf(v, dpp_move<0x4E>(v));
    v = fmaxf(v, dpp_move<0x141>(v));
    v = fmaxf(v, dpp_move<0x140>(v));
    const auto p = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    v = fmaxf(__uint_as_float(p[0]), __uint_as_float(p[1]));
    const auto q = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return fmaxf(__uint_as_float(q[0]), __uint_as_float(q[1]));
}

// Max and sum over the 4 lanes of each DPP quad; every lane of the quad receives the result.
__device__ __forceinline__ float quad_max(float v) {
    v = fmaxf(v, dpp_move<0xB1>(v));
    return fmaxf(v, dpp_move<0x4E>(v));
}
__device__ __forceinline__ float quad_sum(float v) {
    v += dpp_move<0xB1>(v);
    return v + dpp_move<0x4E>(v);
}

// ---------------------------------------------------------------- grouped int8 activations
// Per group of 32 values: scale = max(RN(max|x| / 127), 1e-8), inv = RN(1 / scale),
// q = rint(x * inv) (ties to even), |q| <= 127.  Division here is IEEE (correctly rounded).
__device__ __forceinline__ float g32_scale(float absmax) { return fmaxf(absmax / 127.0f, 1e-8f); }

// Quantize 8 consecutive values into two words in dot4 order: bytes 0..7 hold
// q[0], q[4], q[1], q[5], q[2], q[6], q[3], q[7] -- the order in which (w & 0x0F0F0F0F)
// and ((w >> 4) & 0x0F0F0F0F) expand a row-packed INT4 code word.  Returns the code sum.
// q = rint(v * inv) for inv = RN(1 / scale) of the group's scale (so |v * inv| <= 127 (1 + 3 *
// 2^-24) and |q| <= 127): the product is rounded on its own (kept opaque, so it is not fused
// into the add), then adding 1.5 * 2^23 rounds it to the nearest integer, ties to even, and
// leaves q in the low byte of the result; two byte permutes pack four codes, and the code sum is
// a dot4 of the packed codes with ones.
__device__ __forceinline__ uint32_t pack4_low_bytes(uint32_t a, uint32_t b, uint32_t c, uint32_t d) {
    return __builtin_amdgcn_perm(b, a, 0x0c0c0400u) | (__builtin_amdgcn_perm(d, c, 0x0c0c0400u) << 16);
}

__device__ __forceinline__ int quantize8_dot4(const float* v, float inv, uint32_t& lo, uint32_t& hi) {
    uint32_t t[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        float prod = v[i] * inv;
        asm volatile("" : "+v"(prod));
        t[i] = __float_as_uint(prod + 12582912.0f);
    }
    lo = pack4_low_bytes(t[0], t[4], t[1], t[5]);
    hi = pack4_low_bytes(t[2], t[6], t[3], t[7]);
    return __builtin_amdgcn_sdot4((int)hi, 0x01010101, __builtin_amdgcn_sdot4((int)lo, 0x01010101, 0, false), false);
}

// Byte offset, within its 8-value block, of value t in dot4 order.
__device__ __forceinline__ int dot4_slot(int t) { return ((t & 3) << 1) | (t >> 2); }

// v combined with its lane l ^ 16 / l ^ 32 partner (gfx950 v_permlane16_swap / v_permlane32_swap
// of v with itself: the two results hold, in every lane, the lane's own value and its partner's,
// in an order that depends on the lane; max and + are commutative, so every lane gets the same
// bits as from an exchange through LDS).
__device__ __forceinline__ float max_xor16(float v) {
    const auto p = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return fmaxf(__uint_as_float(p[0]), __uint_as_float(p[1]));
}
__device__ __forceinline__ float max_xor32(float v) {
    const auto p = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return fmaxf(__uint_as_float(p[0]), __uint_as_float(p[1]));
}
__device__ __forceinline__ float sum_xor16(float v) {
    const auto p = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float(p[0]) + __uint_as_float(p[1]);
}
__device__ __forceinline__ float sum_xor32(float v) {
    const auto p = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float(p[0]) + __uint_as_float(p[1]);
}
__device__ __forceinline__ int isum_xor16(int v) {
    const auto p = __builtin_amdgcn_permlane16_swap((unsigned)v, (unsigned)v, false, false);
    return (int)p[0] + (int)p[1];
}

// Max / sum over each 32-lane half of a wave (a group of 32 values, one per lane): the 16-lane
// rows with DPP moves, then one exchange between the two rows of each half.  Both are exact
// (max, integer sum), so the order of the combination does not matter.
__device__ __forceinline__ float half_wave_max(float v) {
    v = fmaxf(v, dpp_move<0xB1>(v));   // quad_perm [1,0,3,2]
    v = fmaxf(v, dpp_move<0x4E>(v));   // quad_perm [2,3,0,1]
    v = fmaxf(v, dpp_move<0x141>(v));  // row_half_mirror
    v = fmaxf(v, dpp_move<0x140>(v));  // row_mirror: every lane holds its row's max
    return max_xor16(v);
}

template <int CTRL>
__device__ __forceinline__ int dpp_move_i(int v) {
    return __builtin_amdgcn_update_dpp(0, v, CTRL, 0xf, 0xf, false);
}

__device__ __forceinline__ int half_wave_sum(int v) {
    v += dpp_move_i<0xB1>(v);
    v += dpp_move_i<0x4E>(v);
    v += dpp_move_i<0x141>(v);
    v += dpp_move_i<0x140>(v);
    return isum_xor16(v);
}

__device__ __forceinline__ float dot2_bf16(uint32_t a, uint32_t b, float c) {
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, a),
                                           __builtin_bit_cast(bf16x2_t, b), c, false);
}

// Constants of dequant_word_mixed.  v_and_or_b32 is a VOP3 form, which on gfx9 takes no literal
// operand and one scalar operand: the masks are pinned in SGPRs, the bias patterns in VGPRs.
// (The two shifts this form saves per word against masking every pair at bits 0..3 measured 2-3%
// on the K = 4096 decode GEMVs.)
struct MixedUnpack {
    uint32_t mask_lo, mask_hi, bf16_bias, f16_bias;
};

__device__ __forceinline__ MixedUnpack make_mixed_unpack() {
    MixedUnpack c{0x000F000Fu, 0x00F000F0u, 0x43004300u, 0x54005400u};
    asm volatile("" : "+s"(c.mask_lo), "+s"(c.mask_hi), "+v"(c.bf16_bias), "+v"(c.f16_bias));
    return c;
}

// The bit-exact bf16 dequant bf16_rne((q - z) * s) of the eight codes of a row-packed word w, as
// four bf16 pairs o[i] = (code 2i, code 2i + 1) (the code of t = 2i at bits [4i, 4i + 4), of
// t = 2i + 1 at bits [16 + 4i, 20 + 4i)).  Each pair is masked in place into a float pair that is
// exact: nibble positions 0 and 4 into bf16 (128 + q) ((w & 0x000F000F) | 0x43004300), positions
// 1 and 5 into fp16 (64 + q) ((w & 0x00F000F0) | 0x54005400: bits 4..7 of the mantissa of 64.0
// weigh 1/16 each, so no shift is needed), and w >> 8 gives positions 2/6 and 3/7 the same way.
// The bf16 pairs meet (s | 0) and (0 | s) in v_dot2_f32_bf16 with bias_bf16 = -(128 + z) s, the
// fp16 halves meet s in v_fma_mix_f32 with bias_f16 = -(64 + z) s: every addend has at most 16
// significant bits, so each fp32 result is exactly (q - z) s, and v_cvt_pk_bf16_f32 rounds each
// pair to nearest even.  The block is one asm statement because a v_dot2 result is not
// interlocked on gfx950: a non-dot VALU may read it only after 3 wait states, which the compiler
// cannot see inside inline asm; here each v_cvt_pk reads v_dot2 results written at least 5
// instructions earlier, and each output register first takes the low product of its pair.
__device__ __forceinline__ void dequant_word_mixed(uint32_t w, const MixedUnpack& c, uint32_t s_lo, uint32_t s_hi,
                                                   float s, float bias_bf16, float bias_f16, uint32_t (&o)[4]) {
    const uint32_t d0 = (w & c.mask_lo) | c.bf16_bias;
    const uint32_t d1 = (w & c.mask_hi) | c.f16_bias;
    const uint32_t w8 = w >> 8;
    const uint32_t d2 = (w8 & c.mask_lo) | c.bf16_bias;
    const uint32_t d3 = (w8 & c.mask_hi) | c.f16_bias;
    float t0, t1, t2, t3;
    asm("v_dot2_f32_bf16 %0, %8, %12, %15\n\t"
        "v_dot2_f32_bf16 %4, %8, %13, %15\n\t"
        "v_dot2_f32_bf16 %2, %10, %12, %15\n\t"
        "v_dot2_f32_bf16 %6, %10, %13, %15\n\t"
        "v_fma_mix_f32 %1, %9, %14, %16 op_sel_hi:[1,0,0]\n\t"
        "v_fma_mix_f32 %5, %9, %14, %16 op_sel:[1,0,0] op_sel_hi:[1,0,0]\n\t"
        "v_fma_mix_f32 %3, %11, %14, %16 op_sel_hi:[1,0,0]\n\t"
        "v_fma_mix_f32 %7, %11, %14, %16 op_sel:[1,0,0] op_sel_hi:[1,0,0]\n\t"
        "v_cvt_pk_bf16_f32 %0, %0, %4\n\t"
        "v_cvt_pk_bf16_f32 %1, %1, %5\n\t"
        "v_cvt_pk_bf16_f32 %2, %2, %6\n\t"
        "v_cvt_pk_bf16_f32 %3, %3, %7"
        : "=&v"(o[0]), "=&v"(o[1]), "=&v"(o[2]), "=&v"(o[3]), "=&v"(t0), "=&v"(t1), "=&v"(t2), "=&v"(t3)
        : "v"(d0), "v"(d1), "v"(d2), "v"(d3), "v"(s_lo), "v"(s_hi), "v"(s), "v"(bias_bf16), "v"(bias_f16));
}

// The group operands of dequant_word_mixed from the scale bits and zero point.  Both biases are
// exact: (128 + z) s and (64 + z) s have at most 16 significant bits, and the fma adds 64 s
// exactly.
struct GroupDequant {
    uint32_t s_lo, s_hi;
    float s, bias_bf16, bias_f16;
};

__device__ __forceinline__ GroupDequant group_dequant(uint32_t s_bits, uint32_t z) {
    GroupDequant g;
    g.s_lo = s_bits & 0xffffu;
    g.s_hi = g.s_lo << 16;
    g.s = __uint_as_float(g.s_lo << 16);
    g.bias_bf16 = -(128.0f + (float)z) * g.s;
    g.bias_f16 = __builtin_fmaf(64.0f, g.s, g.bias_bf16);
    return g;
}

// One 128-dim head through RMSNorm + rotate-half RoPE, one wave per head: lane l holds dims
// l and l + 64 (each other's RoPE partners).  Rounding points of the reference
// (src/moss_tts/_runtime/kernels.py:142-170): xn = bf16(bf16(x * r) * w); out_l =
// bf16(bf16(xn_l * cos_l) + bf16(-xn_{l+64} * sin_l)), out_{l+64} = bf16(bf16(xn_{l+64} *
// cos_{l+64}) + bf16(xn_l * sin_{l+64})), the negation being float negation.
// The squares of a dim pair, contracted one way everywhere (kernels that must agree use this).
__device__ __forceinline__ float head_sq(float a, float b) { return __builtin_fmaf(a, a, b * b); }

// The per-dim part once the head's reciprocal RMS r is known.
__device__ __forceinline__ void head_rope_apply(float a, float b, float r, float w0, float w1, float c0, float c1,
                                                float s0, float s1, uint16_t& o0, uint16_t& o1) {
    const float an = round_bf16(round_bf16(a * r) * w0);
    const float bn = round_bf16(round_bf16(b * r) * w1);
    o0 = f32_to_bf16(round_bf16(an * c0) + round_bf16((-bn) * s0));
    o1 = f32_to_bf16(round_bf16(bn * c1) + round_bf16(an * s1));
}

__device__ __forceinline__ void head_norm_rope(float a, float b, float w0, float w1, float c0, float c1, float s0,
                                               float s1, float eps, uint16_t& o0, uint16_t& o1) {
    const float r = rsqrtf(wave_sum(head_sq(a, b)) / 128.0f + eps);
    head_rope_apply(a, b, r, w0, w1, c0, c1, s0, s1, o0, o1);
}

// The same for one head held by 16 lanes (lane j of the group: dims 4 j .. + 3 in a, their RoPE
// partners 64 + 4 j .. + 3 in b, as 8-byte bf16 quads; weights, cos and sin likewise).  The sum of
// squares follows wave_sum's tree exactly -- pairs and quads inside the lane, then lanes 1 (DPP
// row half mirror), 3 (row mirror), 4 and 8 apart -- so the outputs equal head_norm_rope's bit
// for bit.  All 16 lanes of the group must be active.
__device__ __forceinline__ float xor16(float v, int m) { return __shfl_xor(v, m, 16); }
__device__ __forceinline__ float bf16_quad(uint2 v, int i) {
    return i == 0 ? bf16_lo(v.x) : i == 1 ? bf16_hi(v.x) : i == 2 ? bf16_lo(v.y) : bf16_hi(v.y);
}

__device__ __forceinline__ void head4_norm_rope(uint2 xa, uint2 xb, uint2 wa, uint2 wb, uint2 ca, uint2 cb,
                                                uint2 sa, uint2 sb, float eps, uint2& lo, uint2& hi) {
    float a[4], b[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        a[i] = bf16_quad(xa, i);
        b[i] = bf16_quad(xb, i);
    }
    // stages 1, 2 of wave_sum (lanes 1 and 2 apart there) are this lane's four pairs
    float v = (head_sq(a[0], b[0]) + head_sq(a[1], b[1])) + (head_sq(a[2], b[2]) + head_sq(a[3], b[3]));
    v += xor16(v, 1);  // row_half_mirror: the neighbouring quad
    v += xor16(v, 3);  // row_mirror: the mirrored quad pair (lanes j ^ 2 and j ^ 3 hold the same value)
    v += xor16(v, 4);  // readlanes 0 + 16 and 32 + 48
    v += xor16(v, 8);  // (a + b) + (c + d)
    const float r = rsqrtf(v / 128.0f + eps);
    uint16_t o0[4], o1[4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
        head_rope_apply(a[i], b[i], r, bf16_quad(wa, i), bf16_quad(wb, i), bf16_quad(ca, i), bf16_quad(cb, i),
                        bf16_quad(sa, i), bf16_quad(sb, i), o0[i], o1[i]);
    lo = make_uint2(o0[0] | ((uint32_t)o0[1] << 16), o0[2] | ((uint32_t)o0[3] << 16));
    hi = make_uint2(o1[0] | ((uint32_t)o1[1] << 16), o1[2] | ((uint32_t)o1[3] << 16));
}

}  // namespace moss

// ---------------------------------------------------------------- host-side plumbing
#define MOSS_CHECK_ARG(cond)                                   \
    do {                                                       \
        if (!(cond)) return (int)hipErrorInvalidValue;         \
    } while (0)

#define MOSS_ALIGNED(p, a) ((((uintptr_t)(p)) % (a)) == 0)

static inline int moss_launch_status() { return (int)hipGetLastError(); }

namespace moss {
// norm_rope.hip: the split-K reduction fused with the residual add + RMSNorm after a GEMM.
// The split-K reduction of the QKV GEMM's fp32 partials fused with the q/k-norm + RoPE + KV write
// (cos/sin by position; 8-byte aligned vectors, 16-byte aligned partials).
int qk_rope_from_parts(const float* parts, int S, const void* q_weight, const void* k_weight, const void* cos,
                       const void* sin, void* q_out, void* k_cache, void* v_cache, const void* positions, int L,
                       int ntok, float eps, hipStream_t st);
int addnorm_from_parts(const float* parts, int S, const void* res, const void* w, void* sum_out, void* y, int rows,
                       int n, float eps, hipStream_t st);
// add-RMSNorm of rows x n values in place: xs = bf16(xs + res), y = rmsnorm(xs) (y must not
// overlap xs or res).
int add_rmsnorm_inplace(void* xs, const void* res, const void* w, void* y, int rows, int n, float eps,
                        hipStream_t st);
// w4g32_gemv.hip: 2 .. 4 tokens through the exact GEMV (x bf16 [M, K], y bf16 [M, N], x 16-byte
// aligned), each row of y bit-identical to the single-token GEMV of that token.
bool w4g32_gemv_tokens_shape(int M, int K);
int w4g32_gemv_tokens_launch(const void* x, const void* qw, const void* sc, const void* zp, void* y, int M, int K,
                             int N, hipStream_t st);
}  // namespace moss

// true when the byte ranges [a, a + an) and [b, b + bn) share an address
static inline bool moss_overlaps(const void* a, size_t an, const void* b, size_t bn) {
    const uintptr_t pa = (uintptr_t)a, pb = (uintptr_t)b;
    return pa < pb + bn && pb < pa + an;
}

// The fused-norm projections: res == NULL normalizes x; otherwise s = bf16(x + res) is normalized
// and stored to sum_out by one workgroup while the others still read x and res, so sum_out must not
// overlap either of them (an in-place residual update would race).  K % 2048 == 0, K <= 8192.
static inline int moss_check_norm_args(const void* x, const void* res, const void* norm_w, void* sum_out, int K,
                                       float eps) {
    MOSS_CHECK_ARG(x && norm_w && K > 0 && K % 2048 == 0 && K <= 8192 && eps >= 0.f);
    MOSS_CHECK_ARG((res == nullptr) == (sum_out == nullptr));
    MOSS_CHECK_ARG(MOSS_ALIGNED(x, 16) && MOSS_ALIGNED(norm_w, 16) && MOSS_ALIGNED(res, 16) &&
                   MOSS_ALIGNED(sum_out, 16));
    if (sum_out) {
        const uintptr_t so = (uintptr_t)sum_out, n = (uintptr_t)K * 2;
        MOSS_CHECK_ARG((so + n <= (uintptr_t)x || (uintptr_t)x + n <= so) &&
                       (so + n <= (uintptr_t)res || (uintptr_t)res + n <= so));
    }
    return 0;
}
