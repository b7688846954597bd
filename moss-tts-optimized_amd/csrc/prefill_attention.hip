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
// KV head), KS x 4 waves: wave w takes query head 4 kvh + w % 4 and, of every 64-key block, both
// 32-key halves (KS = 1) or half w / 4 (KS = 2: two waves per head, so each SIMD runs two waves and
// a block's serial chain per wave is halved).  Every K/V block staged in LDS serves all waves.
// Per block, wave and 32-key half:
//   S^T = K Q^T   (32 keys x 32 queries, 8 v_mfma_f32_32x32x16_bf16): with this orientation each
//                 lane holds one query and 16 of its keys, so the row max and sum need one
//                 exchange with the lane 32 away;
//   O^T += V^T P^T (d x queries, 2 x 4 MFMAs): P (rounded to bf16) is the B operand straight from
//                 the S^T registers; the MFMA's K order is permuted to match (the V^T reads use the
//                 same permutation), and O^T keeps one query per lane, so the softmax rescale is a
//                 per-lane factor.
// With KS = 2 the two waves of a head keep their own running max, sum and O^T and are combined once,
// in LDS, at the end (a wave whose keys all lie after a query's position keeps max -inf, sum 0).
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

typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));

// KPT keys per thread (4 with 256 threads, 2 with 512): thread (kg, dc) = (tid / 16, tid % 16)
// holds keys KPT kg .. + KPT - 1 at d 8 dc .. + 7.
template <int KPT>
struct KvRegs {
    u32x4_t k[KPT];
    u32x4_t v[KPT];
};

template <int KPT>
__device__ __forceinline__ void load_kv(KvRegs<KPT>& r, const uint16_t* __restrict__ kc,
                                        const uint16_t* __restrict__ vc, int key0, int tid) {
    const int dc = tid & 15, kg = tid >> 4;
#pragma unroll
    for (int i = 0; i < KPT; ++i) {
        const size_t off = (size_t)(key0 + KPT * kg + i) * kD + 8 * dc;
        r.k[i] = *reinterpret_cast<const u32x4_t*>(kc + off);
        r.v[i] = *reinterpret_cast<const u32x4_t*>(vc + off);
    }
}

__device__ __forceinline__ uint32_t lo_pair(uint32_t a, uint32_t b) { return (a & 0xffffu) | (b << 16); }
__device__ __forceinline__ uint32_t hi_pair(uint32_t a, uint32_t b) { return (a >> 16) | (b & 0xffff0000u); }

// V^T column of key `key` in row d: 8-key groups are swapped by XOR with 8 (d / 32), so that the
// 16 d rows 8 apart that one store instruction writes land in 16 different 4-bank groups (without
// it every V^T store had 4-way bank conflicts, 40% of the kernel's LDS cycles by counters); the
// 32 rows a PV read covers share one d / 32, so the reads keep their layout.  Keeps 4-key groups
// contiguous.
__device__ __forceinline__ int vt_col(int d, int key) { return key ^ (8 * ((d >> 5) & 3)); }

// K rows as they are; V transposed: for each of its 8 d the thread writes its KPT keys as one V^T
// entry (8 bytes for 4 keys, 4 bytes for 2).
template <int KPT>
__device__ __forceinline__ void store_kv(const KvRegs<KPT>& r, uint16_t (*ks)[kKPad], uint16_t (*vt)[kVPad],
                                         int tid) {
    const int dc = tid & 15, kg = tid >> 4;
#pragma unroll
    for (int i = 0; i < KPT; ++i) *reinterpret_cast<u32x4_t*>(&ks[KPT * kg + i][8 * dc]) = r.k[i];
#pragma unroll
    for (int p = 0; p < 4; ++p) {  // d pair 2p, 2p + 1 of the chunk
        if constexpr (KPT == 4) {
            const uint2 even = make_uint2(lo_pair(r.v[0][p], r.v[1][p]), lo_pair(r.v[2][p], r.v[3][p]));
            const uint2 odd = make_uint2(hi_pair(r.v[0][p], r.v[1][p]), hi_pair(r.v[2][p], r.v[3][p]));
            *reinterpret_cast<uint2*>(&vt[8 * dc + 2 * p][vt_col(8 * dc, 4 * kg)]) = even;
            *reinterpret_cast<uint2*>(&vt[8 * dc + 2 * p + 1][vt_col(8 * dc, 4 * kg)]) = odd;
        } else {
            *reinterpret_cast<uint32_t*>(&vt[8 * dc + 2 * p][vt_col(8 * dc, 2 * kg)]) = lo_pair(r.v[0][p], r.v[1][p]);
            *reinterpret_cast<uint32_t*>(&vt[8 * dc + 2 * p + 1][vt_col(8 * dc, 2 * kg)]) = hi_pair(r.v[0][p], r.v[1][p]);
        }
    }
}

template <int KS>
__global__ __launch_bounds__(256 * KS, 1) void prefill_attention_kernel(const uint16_t* __restrict__ q,
                                                                       const uint16_t* __restrict__ k_cache,
                                                                       const uint16_t* __restrict__ v_cache,
                                                                       const int64_t* __restrict__ start,
                                                                       uint16_t* __restrict__ out, int n, int L) {
    constexpr int KPT = 4 / KS;  // keys per thread in the K/V copy
    constexpr int NH = 2 / KS;   // 32-key halves per wave and block
    __shared__ __attribute__((aligned(16))) uint16_t ks[kBK][kKPad];
    __shared__ __attribute__((aligned(16))) uint16_t vt[kD][kVPad];
    __shared__ float xo[KS == 2 ? 4 : 1][KS == 2 ? 66 : 1][64];  // KS = 2: O^T, max, sum of each head's 2nd wave
    const int tid = threadIdx.x, lane = tid & 63, half = lane >> 5, ql = lane & 31;
    const int wave = tid >> 6, hw = wave & 3, kh = KS == 2 ? wave >> 2 : 0;
    const int kvh = blockIdx.y, qh = 4 * kvh + hw;
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

    KvRegs<KPT> kv;
    load_kv<KPT>(kv, kc, vc, 0, tid);
    for (int b = 0; b < nblk; ++b) {
        __syncthreads();  // the previous block's LDS reads are done
        store_kv<KPT>(kv, ks, vt, tid);
        __syncthreads();
        if (b + 1 < nblk) load_kv<KPT>(kv, kc, vc, kBK * (b + 1), tid);

        // S^T for this wave's 32-key halves st = NH kh .. of the block
        f32x16_t s[NH];
#pragma unroll
        for (int h = 0; h < NH; ++h) {
            const int st = NH * kh + h;
#pragma unroll
            for (int e = 0; e < 16; ++e) s[h][e] = 0.f;
#pragma unroll
            for (int kk = 0; kk < 8; ++kk) {
                const bf16x8_t kf = *reinterpret_cast<const bf16x8_t*>(&ks[32 * st + ql][16 * kk + 8 * half]);
                s[h] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kf, qf[kk], s[h], 0, 0, 0);
            }
        }
        // element e of half st: key 64 b + 32 st + 8 (e / 4) + 4 half + e % 4, query ql
        const bool mask = b >= first_masked;
        float bmax = -INFINITY;
#pragma unroll
        for (int h = 0; h < NH; ++h)
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                float v = s[h][e] * c;
                if (mask) {
                    const int key = kBK * b + 32 * (NH * kh + h) + 8 * (e >> 2) + 4 * half + (e & 3);
                    v = key <= qpos ? v : -INFINITY;
                }
                s[h][e] = v;
                bmax = fmaxf(bmax, v);
            }
        bmax = fmaxf(bmax, __shfl_xor(bmax, 32));
        const float mn = fmaxf(m, bmax);
        const float mr = mn == -INFINITY ? 0.f : mn;  // no key of this wave visible yet: nothing changes
        const float alpha = __builtin_amdgcn_exp2f(m - mr);
        m = mn;
        float bsum = 0.f;
        bf16x8_t pf[NH][2];
#pragma unroll
        for (int h = 0; h < NH; ++h)
#pragma unroll
            for (int u = 0; u < 2; ++u)
#pragma unroll
                for (int v = 0; v < 8; ++v) {
                    const float p = __builtin_amdgcn_exp2f(s[h][8 * u + v] - mr);
                    bsum += p;
                    pf[h][u][v] = (__bf16)p;
                }
        bsum += __shfl_xor(bsum, 32);
        l = l * alpha + bsum;
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int e = 0; e < 16; ++e) o[i][e] *= alpha;
        // O^T += V^T P^T: K step (st, u) covers keys 32 st + 16 u + {4 half + 0..3, 8 + 4 half + 0..3}
#pragma unroll
        for (int h = 0; h < NH; ++h)
#pragma unroll
            for (int u = 0; u < 2; ++u) {
                const int key = 32 * (NH * kh + h) + 16 * u + 4 * half;
#pragma unroll
                for (int dt = 0; dt < 4; ++dt) {
                    const uint16_t* row = vt[32 * dt + ql];
                    const uint2 a0 = *reinterpret_cast<const uint2*>(row + vt_col(32 * dt, key));
                    const uint2 a1 = *reinterpret_cast<const uint2*>(row + vt_col(32 * dt, key + 8));
                    const uint4 av = make_uint4(a0.x, a0.y, a1.x, a1.y);
                    o[dt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, av), pf[h][u],
                                                                    o[dt], 0, 0, 0);
                }
            }
    }
    float f1 = 1.f, f2 = 0.f, inv;
    if constexpr (KS == 2) {
        // the two waves of each head meet: the second hands its state to the first through LDS
        if (kh == 1) {
#pragma unroll
            for (int dt = 0; dt < 4; ++dt)
#pragma unroll
                for (int e = 0; e < 16; ++e) xo[hw][16 * dt + e][lane] = o[dt][e];
            xo[hw][64][lane] = m;
            xo[hw][65][lane] = l;
        }
        __syncthreads();
        if (kh == 1) return;
        const float m2 = xo[hw][64][lane], l2 = xo[hw][65][lane];
        const float mx = fmaxf(m, m2);  // finite: key 0 lies in the first wave's half, visible to all
        f1 = __builtin_amdgcn_exp2f(m - mx);
        f2 = __builtin_amdgcn_exp2f(m2 - mx);
        inv = 1.0f / (l * f1 + l2 * f2);
    } else {
        inv = 1.0f / l;  // key 0 is visible to every query
    }
    if (t0 + ql >= n) return;
    uint16_t* orow = out + ((size_t)(t0 + ql) * kQH + qh) * kD;
    // O^T element e of d tile dt: d = 32 dt + 8 (e / 4) + 4 half + e % 4
#pragma unroll
    for (int dt = 0; dt < 4; ++dt)
#pragma unroll
        for (int bq = 0; bq < 4; ++bq) {
            const int d = 32 * dt + 8 * bq + 4 * half;
            float v[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                float a = o[dt][4 * bq + i];
                if constexpr (KS == 2) a = a * f1 + xo[hw][16 * dt + 4 * bq + i][lane] * f2;
                v[i] = a * inv;
            }
            uint2 w;
            w.x = pack_bf16x2(v[0], v[1]);
            w.y = pack_bf16x2(v[2], v[3]);
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
    // measured on MI355X: two waves per head for 128..1024 tokens (up to 256 workgroups, one per CU):
    // at start 0, 256 / 512 / 1024 tokens in 12.6 / 19.6 / 34.3 us against 13.6 / 22.8 / 41.8, and
    // 128 tokens after 1900 cached rows in 60 against 77 us (128 at start 0: 9.2 against 9.0); one
    // wave per head below 128 tokens (64: 6.8 against 7.5 us) and for wider grids (2048: 109 either)
    if (n >= 128 && n <= 1024)
        hipLaunchKernelGGL(prefill_attention_kernel<2>, grid, dim3(512), 0, (hipStream_t)stream, (const uint16_t*)q,
                           (const uint16_t*)k_cache, (const uint16_t*)v_cache, (const int64_t*)start,
                           (uint16_t*)out, n, L);
    else
        hipLaunchKernelGGL(prefill_attention_kernel<1>, grid, dim3(256), 0, (hipStream_t)stream, (const uint16_t*)q,
                           (const uint16_t*)k_cache, (const uint16_t*)v_cache, (const int64_t*)start,
                           (uint16_t*)out, n, L);
    return moss_launch_status();
}
