// Causal GQA attention for the prompt pass (prefill) on the matrix cores.
//
// Qwen3-8B: 32 query heads, 8 KV heads (query head h reads KV head h / 4), head_dim 128, scale
// 1/sqrt(128).  The n prompt tokens sit at absolute positions p0 .. p0 + n - 1 of the static
// cache (their K/V rows already written by the q/k-norm + RoPE kernel); token t attends cache
// rows 0 .. p0 + t.  Output o[t][h * 128 + d] bf16, the O projection's input.
// Reference: F.scaled_dot_product_attention(q, k, v, is_causal=True, scale, enable_gqa=True) of the
// prefill forward (src/moss_tts/_runtime/llm.py:116-128), over the cache rows the prefill wrote
// (llm.py:204-207, prefill_qkv.py:31-53).
//
// Tiling (flash-attention style, online softmax in fp32): one workgroup per (32-token query tile,
// KV head); its 4 waves are the 4 query heads sharing that KV head, so every K/V block staged in
// LDS serves all four.  K/V blocks of 64 keys; per block and wave:
//   S^T = K Q^T   (keys x queries, 2 x 8 v_mfma_f32_32x32x16_bf16): with this orientation each lane
//                 holds one query and 16 of its keys per 32-key half, so the row max and sum need
//                 one exchange with the lane 32 away;
//   O^T += V^T P^T (d x queries, 4 x 4 MFMAs): P (rounded to bf16) is the B operand straight from the
//                 S^T registers; the MFMA's K order is permuted to match (the V^T reads use the same
//                 permutation), and O^T keeps one query per lane, so the softmax rescale is a
//                 per-lane factor.
// V is stored transposed in LDS (V^T[d][key]) so the A operand is two 8-byte reads per MFMA.
// The next K/V block is loaded into registers (ext vectors, so they stay out of scratch) while the
// current one is consumed from LDS.
#include "common.h"

namespace moss {
namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));

constexpr int kQH = 32, kKH = 8, kD = 128;
constexpr int kBQ = 32;              // query tokens per workgroup
constexpr int kBK = 64;              // keys per block
constexpr int kKPad = kD + 8;        // K rows in LDS (bf16), padded
constexpr int kVPad = kBK + 4;       // V^T rows in LDS (bf16), padded

constexpr int kRing = 1;             // K/V blocks in flight per thread (2 and 3 measured no faster at
                                     // 512 tokens, slower at 2048: more VGPRs, one workgroup per CU)

typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));

struct KvRegs {
    u32x4_t k[4];  // 4 x 8 d of keys (tid / 16) * 4 .. + 3 at d 8 (tid % 16)
    u32x4_t v[4];
};

__device__ __forceinline__ void load_kv(KvRegs& r, const uint16_t* __restrict__ kc, const uint16_t* __restrict__ vc,
                                        int key0, int tid) {
    const int dc = tid & 15, kg = tid >> 4;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const size_t off = (size_t)(key0 + 4 * kg + i) * kD + 8 * dc;
        r.k[i] = *reinterpret_cast<const u32x4_t*>(kc + off);
        r.v[i] = *reinterpret_cast<const u32x4_t*>(vc + off);
    }
}

__device__ __forceinline__ uint32_t lo_pair(uint32_t a, uint32_t b) { return (a & 0xffffu) | (b << 16); }
__device__ __forceinline__ uint32_t hi_pair(uint32_t a, uint32_t b) { return (a >> 16) | (b & 0xffff0000u); }

// K rows as they are; V transposed: thread (kg, dc) holds keys 4 kg .. + 3 at d 8 dc .. + 7 and writes,
// for each of its 8 d, the 4 keys as one 8-byte V^T entry.
__device__ __forceinline__ void store_kv(const KvRegs& r, uint16_t (*ks)[kKPad], uint16_t (*vt)[kVPad], int tid) {
    const int dc = tid & 15, kg = tid >> 4;
#pragma unroll
    for (int i = 0; i < 4; ++i) *reinterpret_cast<u32x4_t*>(&ks[4 * kg + i][8 * dc]) = r.k[i];
    const uint32_t w[4][4] = {{r.v[0][0], r.v[0][1], r.v[0][2], r.v[0][3]},
                              {r.v[1][0], r.v[1][1], r.v[1][2], r.v[1][3]},
                              {r.v[2][0], r.v[2][1], r.v[2][2], r.v[2][3]},
                              {r.v[3][0], r.v[3][1], r.v[3][2], r.v[3][3]}};
#pragma unroll
    for (int p = 0; p < 4; ++p) {  // d pair 2p, 2p + 1 of the chunk
        const uint2 even = make_uint2(lo_pair(w[0][p], w[1][p]), lo_pair(w[2][p], w[3][p]));
        const uint2 odd = make_uint2(hi_pair(w[0][p], w[1][p]), hi_pair(w[2][p], w[3][p]));
        *reinterpret_cast<uint2*>(&vt[8 * dc + 2 * p][4 * kg]) = even;
        *reinterpret_cast<uint2*>(&vt[8 * dc + 2 * p + 1][4 * kg]) = odd;
    }
}

__global__ __launch_bounds__(256, 1) void prefill_attention_kernel(const uint16_t* __restrict__ q,
                                                                 const uint16_t* __restrict__ k_cache,
                                                                 const uint16_t* __restrict__ v_cache,
                                                                 const int64_t* __restrict__ start,
                                                                 uint16_t* __restrict__ out, int n, int L) {
    __shared__ __attribute__((aligned(16))) uint16_t ks[kBK][kKPad];
    __shared__ __attribute__((aligned(16))) uint16_t vt[kD][kVPad];
    const int tid = threadIdx.x, lane = tid & 63, half = lane >> 5, ql = lane & 31;
    const int wave = tid >> 6;
    const int kvh = blockIdx.y, qh = 4 * kvh + wave;
    const int t0 = blockIdx.x * kBQ;
    const int64_t p0 = min(max(*start, (int64_t)0), (int64_t)(L - n));
    const int t = min(t0 + ql, n - 1);           // this lane's query token (clamped: stores are guarded)
    const int qpos = (int)p0 + t;                // its absolute position: keys 0 .. qpos
    const int last = (int)p0 + min(t0 + kBQ - 1, n - 1);
    const int nblk = last / kBK + 1;
    const int first_masked = ((int)p0 + t0) / kBK;  // blocks before it hold no key after any query
    const uint16_t* kc = k_cache + (size_t)kvh * L * kD;
    const uint16_t* vc = v_cache + (size_t)kvh * L * kD;

    // Q^T operand: lane holds query ql, d = 16 kk + 8 half .. + 7
    bf16x8_t qf[8];
    {
        const uint16_t* qr = q + ((size_t)t * kQH + qh) * kD + 8 * half;
#pragma unroll
        for (int kk = 0; kk < 8; ++kk) qf[kk] = *reinterpret_cast<const bf16x8_t*>(qr + 16 * kk);
    }
    f32x16_t o[4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int e = 0; e < 16; ++e) o[i][e] = 0.f;
    float m = -INFINITY, l = 0.f;
    const float c = 0.08838834764831845f * 1.4426950408889634f;  // 1/sqrt(128) * log2(e)

    // K/V blocks travel kRing blocks ahead in registers (block b in ring slot b % kRing), so a
    // block's global loads have kRing - 1 blocks of work to arrive
    KvRegs ring[kRing];
#pragma unroll
    for (int i = 0; i < kRing; ++i)
        if (i < nblk) load_kv(ring[i], kc, vc, kBK * i, tid);
    for (int b0 = 0; b0 < nblk; b0 += kRing)
#pragma unroll
    for (int slot = 0; slot < kRing; ++slot) {
        const int b = b0 + slot;
        if (b >= nblk) break;  // uniform
        __syncthreads();  // the previous block's LDS reads are done
        store_kv(ring[slot], ks, vt, tid);
        __syncthreads();
        if (b + kRing < nblk) load_kv(ring[slot], kc, vc, kBK * (b + kRing), tid);

        // S^T for the two 32-key halves of the block
        f32x16_t s[2];
#pragma unroll
        for (int st = 0; st < 2; ++st) {
#pragma unroll
            for (int e = 0; e < 16; ++e) s[st][e] = 0.f;
#pragma unroll
            for (int kk = 0; kk < 8; ++kk) {
                const bf16x8_t kf = *reinterpret_cast<const bf16x8_t*>(&ks[32 * st + ql][16 * kk + 8 * half]);
                s[st] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kf, qf[kk], s[st], 0, 0, 0);
            }
        }
        // element e of half st: key 64 b + 32 st + 8 (e / 4) + 4 half + e % 4, query ql
        const bool mask = b >= first_masked;
        float bmax = -INFINITY;
#pragma unroll
        for (int st = 0; st < 2; ++st)
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                float v = s[st][e] * c;
                if (mask) {
                    const int key = kBK * b + 32 * st + 8 * (e >> 2) + 4 * half + (e & 3);
                    v = key <= qpos ? v : -INFINITY;
                }
                s[st][e] = v;
                bmax = fmaxf(bmax, v);
            }
        bmax = fmaxf(bmax, __shfl_xor(bmax, 32));
        const float mn = fmaxf(m, bmax);            // finite: key 0 is visible to every query
        const float alpha = __builtin_amdgcn_exp2f(m - mn);
        m = mn;
        float bsum = 0.f;
        bf16x8_t pf[2][2];
#pragma unroll
        for (int st = 0; st < 2; ++st)
#pragma unroll
            for (int u = 0; u < 2; ++u)
#pragma unroll
                for (int v = 0; v < 8; ++v) {
                    const float p = __builtin_amdgcn_exp2f(s[st][8 * u + v] - mn);
                    bsum += p;
                    pf[st][u][v] = (__bf16)p;
                }
        bsum += __shfl_xor(bsum, 32);
        l = l * alpha + bsum;
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int e = 0; e < 16; ++e) o[i][e] *= alpha;
        // O^T += V^T P^T: K step (st, u) covers keys 32 st + 16 u + {4 half + 0..3, 8 + 4 half + 0..3}
#pragma unroll
        for (int st = 0; st < 2; ++st)
#pragma unroll
            for (int u = 0; u < 2; ++u) {
                const int key = 32 * st + 16 * u + 4 * half;
#pragma unroll
                for (int dt = 0; dt < 4; ++dt) {
                    const uint16_t* row = vt[32 * dt + ql];
                    const uint2 a0 = *reinterpret_cast<const uint2*>(row + key);
                    const uint2 a1 = *reinterpret_cast<const uint2*>(row + key + 8);
                    const uint4 av = make_uint4(a0.x, a0.y, a1.x, a1.y);
                    o[dt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, av), pf[st][u], o[dt],
                                                                    0, 0, 0);
                }
            }
    }
    if (t0 + ql >= n) return;
    const float inv = 1.0f / l;
    uint16_t* orow = out + ((size_t)(t0 + ql) * kQH + qh) * kD;
    // O^T element e of d tile dt: d = 32 dt + 8 (e / 4) + 4 half + e % 4
#pragma unroll
    for (int dt = 0; dt < 4; ++dt)
#pragma unroll
        for (int bq = 0; bq < 4; ++bq) {
            const int d = 32 * dt + 8 * bq + 4 * half;
            uint2 w;
            w.x = pack_bf16x2(o[dt][4 * bq] * inv, o[dt][4 * bq + 1] * inv);
            w.y = pack_bf16x2(o[dt][4 * bq + 2] * inv, o[dt][4 * bq + 3] * inv);
            *reinterpret_cast<uint2*>(orow + d) = w;
        }
}

}  // namespace
}  // namespace moss

using namespace moss;

MOSS_API int moss_prefill_attention(const void* q, const void* k_cache, const void* v_cache, const void* start,
                                    void* out, int n, int L, void* stream) {
    MOSS_CHECK_ARG(q && k_cache && v_cache && start && out && n > 0 && L > 0 && L % 64 == 0 && n <= L &&
                   L <= 32768);
    MOSS_CHECK_ARG(MOSS_ALIGNED(q, 16) && MOSS_ALIGNED(k_cache, 16) && MOSS_ALIGNED(v_cache, 16) &&
                   MOSS_ALIGNED(start, 8) && MOSS_ALIGNED(out, 8));
    const dim3 grid((unsigned)((n + kBQ - 1) / kBQ), (unsigned)kKH);
    hipLaunchKernelGGL(prefill_attention_kernel, grid, dim3(256), 0, (hipStream_t)stream, (const uint16_t*)q,
                       (const uint16_t*)k_cache, (const uint16_t*)v_cache, (const int64_t*)start, (uint16_t*)out, n,
                       L);
    return moss_launch_status();
}
