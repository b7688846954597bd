// Batch-1 GQA decode attention over a static bf16 KV cache (flash-decoding split + LSE merge)
// and the 33-row embedding sum that starts a decode step.
//
// Semantics of src/moss_tts/_runtime/kernels.py:173-208 (_decode_attn / _decode_attn_reduce):
// scores q.k * 1/sqrt(128) over cache rows t <= p, per split m = max, e = exp(s - m),
// partial = sum(e v) / sum(e), lse = m + log(sum(e)); the merge weights each split by
// exp(lse - max lse) / sum.  Query head h reads KV head h / 4 (32 query, 8 KV heads).
#include "common.h"

namespace moss {
namespace {

constexpr int kHeadDim = 128;
constexpr int kQHeads = 32;
constexpr int kKvHeads = 8;
constexpr int kGroup = kQHeads / kKvHeads;  // 4 query heads per KV head
constexpr int kSplit = 64;                  // cache rows per workgroup
constexpr float kScale = 0.08838834764831845f;

constexpr int kMaxSplits = 512;             // L <= 32768

// grid (8 KV heads, S splits), 256 threads; wave w owns cache rows t0 + 16 w .. + 15 of the
// split's 64.  Each wave loads its K rows as the A operand of v_mfma_f32_16x16x32_bf16 (lane l:
// row l % 16, dims 8 (l / 16) .. + 7 of each 32-dim chunk) and its V rows one 256-byte row per
// load (lane l: dims 2l, 2l + 1), all before any arithmetic, straight into registers.  The scores
// of the 4 query heads are 4 MFMAs (B: the heads' q, columns 4..15 zero); the wave's softmax over
// its 16 rows and its P.V (fp32) need no barrier; the 4 waves' (max, sum, P.V) meet once in LDS,
// rescaled to the split's max.  Each split writes its normalized partial output and log-sum-exp;
// splits after the position write nothing.
//
// FUSED: q, k and v come raw from the q||k||v projection row.  Every workgroup puts its 4
// query heads through head RMSNorm + RoPE (row `position` of the cos/sin tables); the one
// workgroup whose split holds the position also forms the new K row (k-norm + RoPE) and V row,
// stores both into the cache and uses them in place of the cache row it loaded, so no
// workgroup reads a row another one writes (src/moss_tts/_runtime/kernels.py:142-170,211-251).
struct QkvArgs {
    const uint16_t* __restrict__ qnw;  // q head-norm weight [128]
    const uint16_t* __restrict__ knw;  // k head-norm weight [128]
    const uint16_t* __restrict__ cos_t;
    const uint16_t* __restrict__ sin_t;  // [L, 128] tables, row = position
    float eps;
};

typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
constexpr int kWaveRows = kSplit / 4;  // cache rows per wave

template <bool FUSED>
__global__ __launch_bounds__(256) void decode_attn_split(const uint16_t* __restrict__ q,
                                                         uint16_t* __restrict__ kc, uint16_t* __restrict__ vc,
                                                         const int64_t* __restrict__ pos, float* __restrict__ part,
                                                         float* __restrict__ lse, int L, int S, QkvArgs qa) {
    __shared__ __attribute__((aligned(16))) uint16_t qb[kGroup][kHeadDim];  // the 4 query heads, bf16
    __shared__ __attribute__((aligned(16))) uint16_t newkv[2][kHeadDim];     // owner: the new K and V rows
    __shared__ __attribute__((aligned(16))) float pw[4][kGroup][kWaveRows];  // per wave: P[head][row]
    __shared__ __attribute__((aligned(16))) float ow[4][kGroup][kHeadDim];   // per wave: unnormalized P.V
    __shared__ float mw[4][kGroup], lw[4][kGroup];
    const int hk = blockIdx.x, split = blockIdx.y, tid = threadIdx.x;
    const int w = tid / kWave, l = tid & (kWave - 1);
    // rows [0, p] are attended; a position beyond the cache is clamped to its last row (the
    // host API rejects it first; the clamp keeps every access inside the cache regardless)
    const int p = (int)min(max(pos[0], (int64_t)0), (int64_t)(L - 1));
    const int t0 = split * kSplit;
    if (t0 > p) return;  // uniform over the workgroup
    const bool owner = FUSED && p < t0 + kSplit;  // this split holds the new row (uniform)
    const int r0 = t0 + kWaveRows * w;            // this wave's first row
    const bool live = r0 <= p;                    // wave-uniform: the wave holds attended rows

    // Loads, in this order: the q path's (L2 hits; the new K and V rows only by the owner's waves
    // 0 and 1, which form them), then the wave's K and V rows.  Completions are counted in order,
    // so the head norm + RoPE runs while the rows arrive.
    constexpr int D = kHeadDim;
    uint16_t qx0 = 0, qx1 = 0, qw0 = 0, qw1 = 0, cs0 = 0, cs1 = 0, sn0 = 0, sn1 = 0;
    uint16_t kx0 = 0, kx1 = 0, kw0 = 0, kw1 = 0, vx0 = 0, vx1 = 0;
    uint32_t qpair = 0;
    if constexpr (FUSED) {
        // wave w: query head 4 hk + w; lane l: dims l and l + 64
        const uint16_t* cr = qa.cos_t + (size_t)p * D;
        const uint16_t* sr = qa.sin_t + (size_t)p * D;
        const uint16_t* qh = q + (size_t)(hk * kGroup + w) * D;
        const uint16_t* kh = q + (size_t)(kQHeads + hk) * D;
        const uint16_t* vh = q + (size_t)(kQHeads + kKvHeads + hk) * D;
        qx0 = qh[l]; qx1 = qh[l + 64];
        qw0 = qa.qnw[l]; qw1 = qa.qnw[l + 64];
        cs0 = cr[l]; cs1 = cr[l + 64];
        sn0 = sr[l]; sn1 = sr[l + 64];
        if (owner && w == 0) {
            kx0 = kh[l]; kx1 = kh[l + 64];
            kw0 = qa.knw[l]; kw1 = qa.knw[l + 64];
        }
        if (owner && w == 1) {
            vx0 = vh[l]; vx1 = vh[l + 64];
        }
    } else {
        qpair = reinterpret_cast<const uint32_t*>(q + (size_t)hk * kGroup * kHeadDim)[tid];
    }
    __builtin_amdgcn_sched_barrier(0);
    // rows r0 .. r0 + 15 lie inside the cache (t0 <= p < L and L % 64 == 0)
    u32x4_t ka[4] = {};
    uint32_t vv[kWaveRows] = {};
    if (live) {
        const uint16_t* kr = kc + ((size_t)hk * L + r0 + (l & 15)) * D + 8 * (l >> 4);
#pragma unroll
        for (int c = 0; c < 4; ++c) ka[c] = *reinterpret_cast<const u32x4_t*>(kr + 32 * c);
        const uint32_t* vr = reinterpret_cast<const uint32_t*>(vc + ((size_t)hk * L + r0) * D) + l;
#pragma unroll
        for (int r = 0; r < kWaveRows; ++r) vv[r] = vr[r * (D / 2)];
    }
    __builtin_amdgcn_sched_barrier(0);
    if constexpr (FUSED) {
        const float c0 = bf16_bits(cs0), c1 = bf16_bits(cs1);
        const float s0 = bf16_bits(sn0), s1 = bf16_bits(sn1);
        uint16_t o0, o1;
        head_norm_rope(bf16_bits(qx0), bf16_bits(qx1), bf16_bits(qw0), bf16_bits(qw1), c0, c1, s0, s1, qa.eps, o0,
                       o1);
        qb[w][l] = o0;
        qb[w][l + 64] = o1;
        if (owner && w == 0) {  // the new K row of this KV head, into the cache
            uint16_t nk0, nk1;
            head_norm_rope(bf16_bits(kx0), bf16_bits(kx1), bf16_bits(kw0), bf16_bits(kw1), c0, c1, s0, s1, qa.eps,
                           nk0, nk1);
            uint16_t* kd = kc + ((size_t)hk * L + p) * D;
            kd[l] = nk0;
            kd[l + 64] = nk1;
            newkv[0][l] = nk0;
            newkv[0][l + 64] = nk1;
        } else if (owner && w == 1) {  // the new V row (a copy), into the cache
            uint16_t* vd = vc + ((size_t)hk * L + p) * D;
            vd[l] = vx0;
            vd[l + 64] = vx1;
            newkv[1][l] = vx0;
            newkv[1][l + 64] = vx1;
        }
    } else {
        reinterpret_cast<uint32_t*>(&qb[0][0])[tid] = qpair;
    }
    __syncthreads();
    if (owner && p >= r0 && p < r0 + kWaveRows) {  // the new row replaces the stale cache row loaded above
        if (r0 + (l & 15) == p) {
#pragma unroll
            for (int c = 0; c < 4; ++c) ka[c] = *reinterpret_cast<const u32x4_t*>(&newkv[0][32 * c + 8 * (l >> 4)]);
        }
#pragma unroll
        for (int r = 0; r < kWaveRows; ++r)
            if (r0 + r == p) vv[r] = reinterpret_cast<const uint32_t*>(&newkv[1][0])[l];
    }
    // rows after the position never enter P.V (their cache contents are arbitrary)
#pragma unroll
    for (int r = 0; r < kWaveRows; ++r) vv[r] = r0 + r <= p ? vv[r] : 0u;

    // scores: D[row][head] = K q^T; lane l holds rows 4 (l / 16) + i of head l % 16 (heads 4..15 zero)
    const int hd = l & 15;
    f32x4_t sc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int c = 0; c < 4; ++c) {
        const u32x4_t qv = *reinterpret_cast<const u32x4_t*>(&qb[hd & 3][32 * c + 8 * (l >> 4)]);
        const u32x4_t zero = {0u, 0u, 0u, 0u};
        const u32x4_t bq = hd < kGroup ? qv : zero;
        sc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, ka[c]),
                                                     __builtin_bit_cast(bf16x8_t, bq), sc, 0, 0, 0);
    }
    // softmax over the wave's 16 rows, per head: the 4 lanes l % 16 == h hold them
    float sv[4], m = -INFINITY;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int t = r0 + 4 * (l >> 4) + i;
        sv[i] = t <= p ? sc[i] * kScale : -INFINITY;
        m = fmaxf(m, sv[i]);
    }
    m = max_xor32(max_xor16(m));
    float e[4], sum = 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        e[i] = live ? expf(sv[i] - m) : 0.f;  // a live wave's max is finite (row r0 <= p)
        sum += e[i];
    }
    sum = sum_xor32(sum_xor16(sum));
    if (hd < kGroup) *reinterpret_cast<float4*>(&pw[w][hd][4 * (l >> 4)]) = make_float4(e[0], e[1], e[2], e[3]);
    if (l < kGroup) {
        mw[w][l] = m;
        lw[w][l] = sum;
    }
    // P.V of the wave's rows (the wave reads back what it wrote: no barrier): lane l, dims 2l, 2l + 1
    float o[kGroup][2];
#pragma unroll
    for (int h = 0; h < kGroup; ++h) {
        o[h][0] = 0.f;
        o[h][1] = 0.f;
#pragma unroll
        for (int r4 = 0; r4 < kWaveRows / 4; ++r4) {
            const float4 pe = *reinterpret_cast<const float4*>(&pw[w][h][4 * r4]);
            const float pv[4] = {pe.x, pe.y, pe.z, pe.w};
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                o[h][0] = fmaf(pv[i], bf16_lo(vv[4 * r4 + i]), o[h][0]);
                o[h][1] = fmaf(pv[i], bf16_hi(vv[4 * r4 + i]), o[h][1]);
            }
        }
        *reinterpret_cast<float2*>(&ow[w][h][2 * l]) = make_float2(o[h][0], o[h][1]);
    }
    __syncthreads();
    // the split's result: thread (head tid / 64, dims 2 (tid % 64) ..) rescales the 4 waves' parts
    // to the split's max (wave 0 is live, so it is finite)
    const int h = w;
    float mx = mw[0][h];
#pragma unroll
    for (int v = 1; v < 4; ++v) mx = fmaxf(mx, mw[v][h]);
    float den = 0.f, a0 = 0.f, a1 = 0.f;
#pragma unroll
    for (int v = 0; v < 4; ++v) {
        const float f = mw[v][h] == -INFINITY ? 0.f : expf(mw[v][h] - mx);
        const float2 ov = *reinterpret_cast<const float2*>(&ow[v][h][2 * l]);
        den = fmaf(f, lw[v][h], den);
        a0 = fmaf(f, ov.x, a0);
        a1 = fmaf(f, ov.y, a1);
    }
    const int hq = hk * kGroup + h;
    float* dst = part + ((size_t)hq * S + split) * kHeadDim;
    reinterpret_cast<float2*>(dst)[l] = make_float2(a0 / den, a1 / den);
    if (l == 0) lse[hq * S + split] = mx + logf(den);
}

// grid 32 query heads, 128 threads (one per dim).  The splits holding attended rows are
// weighted by exp(lse - max lse) and summed in split order, with no LDS and no barrier.  The
// first CHUNK splits' partials (CHUNK = 32 for L <= 2048, else 64: L <= 4096) are loaded together
// with the lse values, so a typical merge is one round trip; the split order of the sum does not
// depend on CHUNK.
constexpr int kMergeChunk = 64;

// QUANT: the merged bf16 row also leaves as int8 groups of 32 (4 per head; the groups of a
// wave are its two 32-lane halves), each group's scale max(RN(max|x| / 127), 1e-8), codes
// rint(x * RN(1 / scale)) stored in dot4 order and their sum, as the standalone quantizer forms
// them (src/moss_tts/_runtime/attention_quant.py:8-23).
struct MergeQuant {
    int8_t* __restrict__ qx;
    float* __restrict__ sx;
    int* __restrict__ qsum;
};

template <bool QUANT, int CHUNK>
__global__ __launch_bounds__(128) void decode_attn_merge(const float* __restrict__ part,
                                                         const float* __restrict__ lse,
                                                         const int64_t* __restrict__ pos, uint16_t* __restrict__ out,
                                                         int L, int S, MergeQuant mq) {
    static_assert(CHUNK <= kMergeChunk, "the first chunk's weights come from one lane each");
    const int hq = blockIdx.x, d = threadIdx.x, lane = d & (kWave - 1);
    // the partials and this lane's first lse value are loaded together with the position
    // (clamped into the workspace, branch-free) and masked once the position is known
    const int64_t p_raw = pos[0];
    const float* src = part + (size_t)hq * S * kHeadDim + d;
    float v[CHUNK];
#pragma unroll
    for (int u = 0; u < CHUNK; ++u) v[u] = src[(size_t)min(u, S - 1) * kHeadDim];
    const float lse0 = lse[hq * S + min(lane, S - 1)];
    const int p = (int)min(max(p_raw, (int64_t)0), (int64_t)(L - 1));
    const int active = p / kSplit + 1;
    // each wave covers every split (lane s holds splits s, s + 64, ...): the max, the weights and
    // their sum need no exchange between the two waves
    float mx = lane < active ? lse0 : -INFINITY;
    for (int s = lane + kWave; s < active; s += kWave) mx = fmaxf(mx, lse[hq * S + s]);
    mx = wave_max(mx);
    const float e0 = lane < active ? expf(lse0 - mx) : 0.f;  // the weight of split `lane`
    float ws = e0;
    for (int s = lane + kWave; s < active; s += kWave) ws += expf(lse[hq * S + s] - mx);
    const float wsum = wave_sum(ws);
    float acc = 0.f;
#pragma unroll
    for (int u = 0; u < CHUNK; ++u) {  // split order; split u's weight from lane u
        const float wu = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(e0), u));
        if (u < active) acc = fmaf(wu, v[u], acc);
    }
    for (int s = CHUNK; s < active; ++s) {  // splits 32 .. 63 (CHUNK 32 only) have their weight in lane s
        const float ws_ = s < kWave ? __int_as_float(__builtin_amdgcn_readlane(__float_as_int(e0), s))
                                    : expf(lse[hq * S + s] - mx);
        acc = fmaf(ws_, src[(size_t)s * kHeadDim], acc);
    }
    const uint16_t o = f32_to_bf16(acc / wsum);
    out[hq * kHeadDim + d] = o;
    if constexpr (QUANT) {
        const float x = bf16_bits(o);
        const float scale = g32_scale(half_wave_max(fabsf(x)));
        const int q = (int)rintf(x * (1.0f / scale));
        const int total = half_wave_sum(q);
        const int g = hq * (kHeadDim / 32) + d / 32, t = d & 31;
        mq.qx[g * 32 + 8 * (t >> 3) + dot4_slot(t & 7)] = (int8_t)q;
        if (t == 0) {
            mq.sx[g] = scale;
            mq.qsum[g] = total;
        }
    }
}

template <bool QUANT>
void launch_merge(const float* part, const float* lse, const int64_t* pos, uint16_t* out, int L, int S,
                  const MergeQuant& mq, hipStream_t st) {
    if (S <= 32)
        hipLaunchKernelGGL((decode_attn_merge<QUANT, 32>), dim3(kQHeads), dim3(kHeadDim), 0, st, part, lse, pos, out,
                           L, S, mq);
    else
        hipLaunchKernelGGL((decode_attn_merge<QUANT, kMergeChunk>), dim3(kQHeads), dim3(kHeadDim), 0, st, part, lse,
                           pos, out, L, S, mq);
}

// ids int64 [T, Q+1] (text token, then one code per codebook); grid (T, H / (256 VEC)): each
// thread sums VEC consecutive elements (VEC = 8 / 4: 16- / 8-byte loads, for H % 8 / 4 == 0),
// every element in the same order (text row, then codebooks 0 .. Q-1, bf16 after every add).
// Ids are clamped into their tables so device-side data can never index outside them.
template <int VEC>
__global__ __launch_bounds__(256) void embedding_sum_rows(const int64_t* __restrict__ ids,
                                                          const uint16_t* __restrict__ text,
                                                          const uint16_t* __restrict__ audio,
                                                          uint16_t* __restrict__ out, int H, int Vt, int V, int Q) {
    typedef uint16_t vec_t __attribute__((ext_vector_type(VEC)));
    const int t = blockIdx.x, d = VEC * (blockIdx.y * blockDim.x + threadIdx.x);
    if (d >= H) return;
    const int64_t* row = ids + (size_t)t * (Q + 1);
    const int64_t tok = min(max(row[0], (int64_t)0), (int64_t)(Vt - 1));
    const vec_t x0 = *reinterpret_cast<const vec_t*>(text + (size_t)tok * H + d);
    float x[VEC];
#pragma unroll
    for (int j = 0; j < VEC; ++j) x[j] = bf16_bits(x0[j]);
    // the codebook rows of the usual Q <= 32 are loaded together, then added in order
    constexpr int kBatch = 32;
    for (int q0 = 0; q0 < Q; q0 += kBatch) {
        vec_t a[kBatch];
#pragma unroll
        for (int u = 0; u < kBatch; ++u) {
            const int qi = min(q0 + u, Q - 1);
            const int64_t c = min(max(row[qi + 1], (int64_t)0), (int64_t)(V - 1));
            a[u] = *reinterpret_cast<const vec_t*>(audio + ((size_t)qi * V + c) * H + d);
        }
#pragma unroll
        for (int u = 0; u < kBatch; ++u)
            if (q0 + u < Q)
#pragma unroll
                for (int j = 0; j < VEC; ++j) x[j] = round_bf16(x[j] + bf16_bits(a[u][j]));
    }
    vec_t y;
#pragma unroll
    for (int j = 0; j < VEC; ++j) y[j] = f32_to_bf16(x[j]);
    *reinterpret_cast<vec_t*>(out + (size_t)t * H + d) = y;
}

}  // namespace
}  // namespace moss

using namespace moss;

MOSS_API int moss_decode_attention_splits(int L) { return (L + kSplit - 1) / kSplit; }

MOSS_API int moss_decode_attention(const void* q, const void* k_cache, const void* v_cache, const void* position,
                                   void* partial, void* lse, void* out, int L, void* stream) {
    MOSS_CHECK_ARG(q && k_cache && v_cache && position && partial && lse && out);
    MOSS_CHECK_ARG(L > 0 && L % kSplit == 0 && L / kSplit <= kMaxSplits);
    MOSS_CHECK_ARG(MOSS_ALIGNED(k_cache, 16) && MOSS_ALIGNED(v_cache, 16) && MOSS_ALIGNED(q, 4) &&
                   MOSS_ALIGNED(partial, 8) && MOSS_ALIGNED(out, 2));
    const int S = L / kSplit;
    hipStream_t st = (hipStream_t)stream;
    hipLaunchKernelGGL(decode_attn_split<false>, dim3(kKvHeads, S), dim3(256), 0, st, (const uint16_t*)q,
                       (uint16_t*)k_cache, (uint16_t*)v_cache, (const int64_t*)position, (float*)partial,
                       (float*)lse, L, S, QkvArgs{});
    launch_merge<false>((const float*)partial, (const float*)lse, (const int64_t*)position, (uint16_t*)out, L, S,
                        MergeQuant{}, st);
    return moss_launch_status();
}

namespace {

int attention_qkv(const void* qkv, const void* q_norm_w, const void* k_norm_w, const void* cos_t, const void* sin_t,
                  void* k_cache, void* v_cache, const void* position, void* partial, void* lse, void* out, int L,
                  float eps, const MergeQuant* mq, void* stream) {
    MOSS_CHECK_ARG(qkv && q_norm_w && k_norm_w && cos_t && sin_t && k_cache && v_cache && position && partial &&
                   lse && out && eps >= 0.f);
    MOSS_CHECK_ARG(L > 0 && L % kSplit == 0 && L / kSplit <= kMaxSplits);
    MOSS_CHECK_ARG(MOSS_ALIGNED(k_cache, 16) && MOSS_ALIGNED(v_cache, 16) && MOSS_ALIGNED(qkv, 4) &&
                   MOSS_ALIGNED(partial, 8) && MOSS_ALIGNED(out, 2));
    const int S = L / kSplit;
    hipStream_t st = (hipStream_t)stream;
    const QkvArgs qa{(const uint16_t*)q_norm_w, (const uint16_t*)k_norm_w, (const uint16_t*)cos_t,
                     (const uint16_t*)sin_t, eps};
    hipLaunchKernelGGL(decode_attn_split<true>, dim3(kKvHeads, S), dim3(256), 0, st, (const uint16_t*)qkv,
                       (uint16_t*)k_cache, (uint16_t*)v_cache, (const int64_t*)position, (float*)partial,
                       (float*)lse, L, S, qa);
    if (mq)
        launch_merge<true>((const float*)partial, (const float*)lse, (const int64_t*)position, (uint16_t*)out, L, S,
                           *mq, st);
    else
        launch_merge<false>((const float*)partial, (const float*)lse, (const int64_t*)position, (uint16_t*)out, L, S,
                            MergeQuant{}, st);
    return moss_launch_status();
}

}  // namespace

MOSS_API int moss_decode_attention_qkv(const void* qkv, const void* q_norm_w, const void* k_norm_w, const void* cos_t,
                                       const void* sin_t, void* k_cache, void* v_cache, const void* position,
                                       void* partial, void* lse, void* out, int L, float eps, void* stream) {
    return attention_qkv(qkv, q_norm_w, k_norm_w, cos_t, sin_t, k_cache, v_cache, position, partial, lse, out, L, eps,
                         nullptr, stream);
}

MOSS_API int moss_decode_attention_qkv_quant(const void* qkv, const void* q_norm_w, const void* k_norm_w,
                                             const void* cos_t, const void* sin_t, void* k_cache, void* v_cache,
                                             const void* position, void* partial, void* lse, void* out, void* out_qx,
                                             void* out_sx, void* out_qsum, int L, float eps, void* stream) {
    MOSS_CHECK_ARG(out_qx && out_sx && out_qsum && MOSS_ALIGNED(out_sx, 4) && MOSS_ALIGNED(out_qsum, 4));
    const MergeQuant mq{(int8_t*)out_qx, (float*)out_sx, (int*)out_qsum};
    return attention_qkv(qkv, q_norm_w, k_norm_w, cos_t, sin_t, k_cache, v_cache, position, partial, lse, out, L, eps,
                         &mq, stream);
}

MOSS_API int moss_embedding_sum(const void* ids, const void* text, const void* audio, void* out, int T, int H,
                                int Vt, int V, int Q, void* stream) {
    MOSS_CHECK_ARG(ids && text && audio && out && T > 0 && H > 0 && Vt > 0 && V > 0 && Q >= 0);
    // 16- or 8-byte loads where rows allow them: 512 tokens x 33 rows of 4096 in 50 us with 2-byte loads
    if (H % 8 == 0 && MOSS_ALIGNED(text, 16) && MOSS_ALIGNED(audio, 16) && MOSS_ALIGNED(out, 16))
        hipLaunchKernelGGL(embedding_sum_rows<8>, dim3(T, (H / 8 + 255) / 256), dim3(256), 0, (hipStream_t)stream,
                           (const int64_t*)ids, (const uint16_t*)text, (const uint16_t*)audio, (uint16_t*)out, H, Vt,
                           V, Q);
    else if (H % 4 == 0 && MOSS_ALIGNED(text, 8) && MOSS_ALIGNED(audio, 8) && MOSS_ALIGNED(out, 8))
        hipLaunchKernelGGL(embedding_sum_rows<4>, dim3(T, (H / 4 + 255) / 256), dim3(256), 0, (hipStream_t)stream,
                           (const int64_t*)ids, (const uint16_t*)text, (const uint16_t*)audio, (uint16_t*)out, H, Vt,
                           V, Q);
    else
        hipLaunchKernelGGL(embedding_sum_rows<1>, dim3(T, (H + 255) / 256), dim3(256), 0, (hipStream_t)stream,
                           (const int64_t*)ids, (const uint16_t*)text, (const uint16_t*)audio, (uint16_t*)out, H, Vt,
                           V, Q);
    return moss_launch_status();
}
