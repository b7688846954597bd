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

// grid (8 KV heads, S splits), 256 threads.
__global__ __launch_bounds__(256) void decode_attn_split(const uint16_t* __restrict__ q,
                                                         const uint16_t* __restrict__ kc,
                                                         const uint16_t* __restrict__ vc,
                                                         const int64_t* __restrict__ pos, float* __restrict__ part,
                                                         float* __restrict__ lse, int L, int S) {
    __shared__ float qs[kGroup][kHeadDim];
    __shared__ float pr[kGroup][kSplit];
    __shared__ float denom_s[kGroup];
    const int hk = blockIdx.x, split = blockIdx.y, tid = threadIdx.x;
    // rows [0, p] are attended; a position beyond the cache is clamped to its last row (the
    // host API rejects it first; the clamp keeps every access inside the cache regardless)
    const int p = (int)min(max(pos[0], (int64_t)0), (int64_t)(L - 1));
    const int t0 = split * kSplit;
    if (t0 > p) {  // every row of this split is masked (uniform over the workgroup)
        const int j = tid / kWave, l = tid & (kWave - 1);
        const int hq = hk * kGroup + j;
        part[((size_t)hq * S + split) * kHeadDim + l] = 0.f;
        part[((size_t)hq * S + split) * kHeadDim + l + 64] = 0.f;
        if (l == 0) lse[hq * S + split] = -INFINITY;
        return;
    }
    // the 4 query heads of this KV head, fp32 in LDS
    {
        const uint32_t w = reinterpret_cast<const uint32_t*>(q + (size_t)hk * kGroup * kHeadDim)[tid];
        const int j = (2 * tid) / kHeadDim, d = (2 * tid) % kHeadDim;
        qs[j][d] = bf16_lo(w);
        qs[j][d + 1] = bf16_hi(w);
    }
    __syncthreads();
    // scores: four threads per cache row, each a 32-dim quarter (64 contiguous bytes)
    {
        const int tl = tid >> 2, qd = tid & 3, t = t0 + tl;
        float s0 = 0.f, s1 = 0.f, s2 = 0.f, s3 = 0.f;
        if (t <= p) {
            const uint4* kr = reinterpret_cast<const uint4*>(kc + ((size_t)hk * L + t) * kHeadDim + 32 * qd);
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                const uint4 v = kr[c];
                const uint32_t kw[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const int d = 32 * qd + 8 * c + 2 * e;
                    const float k0 = bf16_lo(kw[e]), k1 = bf16_hi(kw[e]);
                    s0 = fmaf(k1, qs[0][d + 1], fmaf(k0, qs[0][d], s0));
                    s1 = fmaf(k1, qs[1][d + 1], fmaf(k0, qs[1][d], s1));
                    s2 = fmaf(k1, qs[2][d + 1], fmaf(k0, qs[2][d], s2));
                    s3 = fmaf(k1, qs[3][d + 1], fmaf(k0, qs[3][d], s3));
                }
            }
        }
        // sum the four quarters (lanes of one DPP quad)
        s0 += dpp_move<0xB1>(s0); s0 += dpp_move<0x4E>(s0);
        s1 += dpp_move<0xB1>(s1); s1 += dpp_move<0x4E>(s1);
        s2 += dpp_move<0xB1>(s2); s2 += dpp_move<0x4E>(s2);
        s3 += dpp_move<0xB1>(s3); s3 += dpp_move<0x4E>(s3);
        if (qd == 0) {
            const bool ok = t <= p;
            pr[0][tl] = ok ? s0 * kScale : -INFINITY;
            pr[1][tl] = ok ? s1 * kScale : -INFINITY;
            pr[2][tl] = ok ? s2 * kScale : -INFINITY;
            pr[3][tl] = ok ? s3 * kScale : -INFINITY;
        }
    }
    __syncthreads();
    // softmax within the split: wave j handles query head j, lane l cache row t0 + l
    const int j = tid / kWave, l = tid & (kWave - 1);
    float m;
    {
        const float v = pr[j][l];
        m = wave_max(v);                         // finite: row t0 <= p is valid
        const float e = (t0 + l <= p) ? expf(v - m) : 0.f;
        const float d = wave_sum(e);
        pr[j][l] = e;
        if (l == 0) denom_s[j] = d;
    }
    __syncthreads();
    // P.V: lane l owns dims 2l, 2l+1 of query head j
    const int hq = hk * kGroup + j;
    float a0 = 0.f, a1 = 0.f;
    const int rows = min(kSplit, p - t0 + 1);
    const uint32_t* vr = reinterpret_cast<const uint32_t*>(vc + ((size_t)hk * L + t0) * kHeadDim) + l;
#pragma unroll 8
    for (int tl = 0; tl < rows; ++tl) {
        const uint32_t v = vr[(size_t)tl * (kHeadDim / 2)];
        const float e = pr[j][tl];
        a0 = fmaf(e, bf16_lo(v), a0);
        a1 = fmaf(e, bf16_hi(v), a1);
    }
    const float den = denom_s[j];
    float* dst = part + ((size_t)hq * S + split) * kHeadDim;
    dst[2 * l] = a0 / den;
    dst[2 * l + 1] = a1 / den;
    if (l == 0) lse[hq * S + split] = m + logf(den);
}

// grid 32 query heads, 128 threads (one per dim): merge the splits, bf16 out [32 * 128].
__global__ __launch_bounds__(128) void decode_attn_merge(const float* __restrict__ part,
                                                         const float* __restrict__ lse, uint16_t* __restrict__ out,
                                                         int S) {
    const int hq = blockIdx.x, d = threadIdx.x;
    float mx = -INFINITY;
    for (int s = 0; s < S; ++s) mx = fmaxf(mx, lse[hq * S + s]);
    float wsum = 0.f, acc = 0.f;
    for (int s = 0; s < S; ++s) {
        const float w = expf(lse[hq * S + s] - mx);  // exp(-inf) = 0 for masked splits
        wsum += w;
        acc = fmaf(w, part[((size_t)hq * S + s) * kHeadDim + d], acc);
    }
    out[hq * kHeadDim + d] = f32_to_bf16(acc / wsum);
}

// ids int64 [T, Q+1] (text token, then one code per codebook); grid (T, H / 256).
// Ids are clamped into their tables so device-side data can never index outside them.
__global__ __launch_bounds__(256) void embedding_sum_rows(const int64_t* __restrict__ ids,
                                                          const uint16_t* __restrict__ text,
                                                          const uint16_t* __restrict__ audio,
                                                          uint16_t* __restrict__ out, int H, int Vt, int V, int Q) {
    const int t = blockIdx.x, d = blockIdx.y * blockDim.x + threadIdx.x;
    if (d >= H) return;
    const int64_t* row = ids + (size_t)t * (Q + 1);
    const int64_t tok = min(max(row[0], (int64_t)0), (int64_t)(Vt - 1));
    float x = bf16_bits(text[(size_t)tok * H + d]);
    for (int qi = 0; qi < Q; ++qi) {
        const int64_t c = min(max(row[qi + 1], (int64_t)0), (int64_t)(V - 1));
        x = round_bf16(x + bf16_bits(audio[((size_t)qi * V + c) * H + d]));
    }
    out[(size_t)t * H + d] = f32_to_bf16(x);
}

}  // namespace
}  // namespace moss

using namespace moss;

MOSS_API int moss_decode_attention_splits(int L) { return (L + kSplit - 1) / kSplit; }

MOSS_API int moss_decode_attention(const void* q, const void* k_cache, const void* v_cache, const void* position,
                                   void* partial, void* lse, void* out, int L, void* stream) {
    MOSS_CHECK_ARG(q && k_cache && v_cache && position && partial && lse && out && L > 0);
    MOSS_CHECK_ARG(MOSS_ALIGNED(k_cache, 16) && MOSS_ALIGNED(v_cache, 16) && MOSS_ALIGNED(q, 4));
    const int S = (L + kSplit - 1) / kSplit;
    hipStream_t st = (hipStream_t)stream;
    hipLaunchKernelGGL(decode_attn_split, dim3(kKvHeads, S), dim3(256), 0, st, (const uint16_t*)q,
                       (const uint16_t*)k_cache, (const uint16_t*)v_cache, (const int64_t*)position, (float*)partial,
                       (float*)lse, L, S);
    hipLaunchKernelGGL(decode_attn_merge, dim3(kQHeads), dim3(kHeadDim), 0, st, (const float*)partial,
                       (const float*)lse, (uint16_t*)out, S);
    return moss_launch_status();
}

MOSS_API int moss_embedding_sum(const void* ids, const void* text, const void* audio, void* out, int T, int H,
                                int Vt, int V, int Q, void* stream) {
    MOSS_CHECK_ARG(ids && text && audio && out && T > 0 && H > 0 && Vt > 0 && V > 0 && Q >= 0);
    hipLaunchKernelGGL(embedding_sum_rows, dim3(T, (H + 255) / 256), dim3(256), 0, (hipStream_t)stream,
                       (const int64_t*)ids, (const uint16_t*)text, (const uint16_t*)audio, (uint16_t*)out, H, Vt, V,
                       Q);
    return moss_launch_status();
}
