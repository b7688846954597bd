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
// HPW query heads of one KV head), KS waves per head: wave (kq, hw) takes query head hw of the group
// and the 32-key part kq of every block of 32 KS keys, so a block's keys are split over the KS waves
// of a head and the serial chain of blocks is KS times shorter than one wave per head would make
// it.  Shapes: 2 heads x 4 parts (128-key blocks) while 16 workgroups per 32 tokens fill at most
// one per CU, else 4 heads x 2 parts (64-key blocks).  Tiles are issued longest first.
// Every K/V block staged in LDS serves all waves.  Per block and wave:
//   S^T = K Q^T   (32 keys x 32 queries, 8 v_mfma_f32_32x32x16_bf16): with this orientation each
//                 lane holds one query and 16 of its keys, so the row max and sum need one
//                 exchange with the lane 32 away;
//   O^T += V^T P^T (d x queries, 2 x 4 MFMAs): P (rounded to bf16) is the B operand straight from
//                 the S^T registers; the MFMA's K order is permuted to match (the V^T reads use the
//                 same permutation), and O^T keeps one query per lane, so the softmax rescale is a
//                 per-lane factor.
// The KS waves of a head keep their own running max, sum and O^T and are combined once, in LDS, at
// the end: each finishes the d tiles it owns (a wave whose keys all lie after a query's position
// keeps max -inf, sum 0 and O^T 0 for it).
// V is stored transposed in LDS (V^T[d][key]) so the A operand is two 8-byte reads per MFMA.
// K/V blocks go through registers (ext vectors, so they stay out of scratch) into two LDS stages:
// block b + 2 is loaded while block b is consumed and b + 1 waits in the other stage, one barrier
// per block.
#include "common.h"

namespace moss {
namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));

constexpr int kQH = 32, kKH = 8, kD = 128;
constexpr int kBQ = 32;              // query tokens per workgroup
constexpr int kKPad = kD + 8;        // K rows in LDS (bf16), padded

// Workgroup shape: HPW query heads of one KV head, KS waves per head, wave kq taking the 32-key
// part kq of every block of 32 KS keys.
template <int HPW, int KS>
struct Tile {
    static constexpr int kWaves = HPW * KS, kThreads = 64 * kWaves;
    static constexpr int kBK = 32 * KS;                            // keys per block
    static constexpr int kKPT = 16 * kBK / kThreads;               // keys per thread in the K/V copy
    static constexpr int kVPad = kBK + 4;                          // V^T rows in LDS (bf16), padded
    static constexpr int kKBytes = kBK * kKPad * 2;
    static constexpr int kStage = kKBytes + kD * kVPad * 2;        // one K + V^T stage
    static constexpr int kXo = HPW * 4 * (KS - 1) * 4 * 64 * 16;  // O^T tiles handed over
    static constexpr int kMl = HPW * KS * 2 * 64 * 4;              // running max and sum
    static constexpr int kLds = 2 * kStage > kXo + kMl ? 2 * kStage : kXo + kMl;
    static_assert(KS >= 2 && HPW * KS <= 8, "2 to 8 waves, 2 or more per head");
    static_assert(kKPT == 2 || kKPT == 4, "K/V copy takes 2 or 4 keys per thread");
};

typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));

// KPT keys per thread: thread (kg, dc) = (tid / 16, tid % 16) holds keys KPT kg .. + KPT - 1 of
// the block at d 8 dc .. + 7.  Rows after `last` (the last key any query of the tile sees) are
// zeros, not loads: they may lie past the cache or hold rows never written, and a P of 0 times a
// NaN there would still poison O.
template <int KPT>
struct KvRegs {
    u32x4_t k[KPT];
    u32x4_t v[KPT];
};

template <int KPT>
__device__ __forceinline__ void load_kv(KvRegs<KPT>& r, const uint16_t* __restrict__ kc,
                                        const uint16_t* __restrict__ vc, int key0, int last, int tid) {
    const int dc = tid & 15, kg = tid >> 4;
#pragma unroll
    for (int i = 0; i < KPT; ++i) {
        const int key = key0 + KPT * kg + i;
        const size_t off = (size_t)key * kD + 8 * dc;
        const u32x4_t z = {0u, 0u, 0u, 0u};
        r.k[i] = key <= last ? *reinterpret_cast<const u32x4_t*>(kc + off) : z;
        r.v[i] = key <= last ? *reinterpret_cast<const u32x4_t*>(vc + off) : z;
    }
}

__device__ __forceinline__ uint32_t lo_pair(uint32_t a, uint32_t b) { return (a & 0xffffu) | (b << 16); }
__device__ __forceinline__ uint32_t hi_pair(uint32_t a, uint32_t b) { return (a >> 16) | (b & 0xffff0000u); }

// V^T column of key `key` in row d: 8-key groups are swapped by XOR with 8 (d / 32), so that the
// 16 d rows 8 apart that one store instruction writes land in 16 different 4-bank groups (without
// it every V^T store had 4-way bank conflicts, 40% of the kernel's LDS cycles by counters); the
// 32 rows a PV read covers share one d / 32, so the reads keep their layout.  Keeps 4-key groups
// contiguous (and within their 32-key part).
__device__ __forceinline__ int vt_col(int d, int key) { return key ^ (8 * ((d >> 5) & 3)); }

// K rows as they are; V transposed: for each of its 8 d the thread writes its KPT keys as one V^T
// entry (8 bytes for 4 keys, 4 bytes for 2).
template <int KPT, int VPAD>
__device__ __forceinline__ void store_kv(const KvRegs<KPT>& r, uint16_t (*ks)[kKPad], uint16_t (*vt)[VPAD],
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

template <int HPW, int KS>
__global__ __launch_bounds__(64 * HPW * KS, 1) void prefill_attention_kernel(
    const uint16_t* __restrict__ q, const uint16_t* __restrict__ k_cache, const uint16_t* __restrict__ v_cache,
    const int64_t* __restrict__ start, uint16_t* __restrict__ out, int n, int L) {
    using T = Tile<HPW, KS>;
    constexpr int KPT = T::kKPT, BK = T::kBK, VPAD = T::kVPad;
    // two K + V^T stages (block b in stage b % 2: one barrier per block), then the combine area
    __shared__ __attribute__((aligned(16))) unsigned char smem[T::kLds];
    const int tid = threadIdx.x, lane = tid & 63, half = lane >> 5, ql = lane & 31;
    const int wave = tid >> 6, hw = wave % HPW, kq = wave / HPW;
    const int kvh = blockIdx.y / (4 / HPW), qh = 4 * kvh + HPW * (blockIdx.y % (4 / HPW)) + hw;
    const int t0 = (gridDim.x - 1 - blockIdx.x) * kBQ;  // longest tiles first
    const int64_t p0 = min(max(*start, (int64_t)0), (int64_t)(L - n));
    const int t = min(t0 + ql, n - 1);           // this lane's query token (clamped: stores are guarded)
    const int qpos = (int)p0 + t;                // its absolute position: keys 0 .. qpos
    const int last = (int)p0 + min(t0 + kBQ - 1, n - 1);
    const int nblk = last / BK + 1;
    const int first_masked = ((int)p0 + t0) / BK;  // blocks before it hold no key after any query
    const uint16_t* kc = k_cache + (size_t)kvh * L * kD;
    const uint16_t* vc = v_cache + (size_t)kvh * L * kD;
    auto stage_k = [&](int s) { return reinterpret_cast<uint16_t(*)[kKPad]>(smem + s * T::kStage); };
    auto stage_v = [&](int s) { return reinterpret_cast<uint16_t(*)[VPAD]>(smem + s * T::kStage + T::kKBytes); };

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
    load_kv<KPT>(kv, kc, vc, 0, last, tid);
    store_kv<KPT, VPAD>(kv, stage_k(0), stage_v(0), tid);
    if (nblk > 1) load_kv<KPT>(kv, kc, vc, BK, last, tid);
    for (int b = 0; b < nblk; ++b) {
        // block b is staged by every wave, and every wave is done with block b - 1's stage
        __syncthreads();
        const uint16_t(*ks)[kKPad] = stage_k(b & 1);
        const uint16_t(*vt)[VPAD] = stage_v(b & 1);
        if (BK * b + 32 * kq <= last) {  // else every key of this wave's part is masked
            // S^T for this wave's 32-key part of the block
            f32x16_t s = {};
#pragma unroll
            for (int kk = 0; kk < 8; ++kk) {
                const bf16x8_t kf = *reinterpret_cast<const bf16x8_t*>(&ks[32 * kq + ql][16 * kk + 8 * half]);
                s = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kf, qf[kk], s, 0, 0, 0);
            }
            // element e: key BK b + 32 kq + 8 (e / 4) + 4 half + e % 4, query ql
            const bool mask = b >= first_masked;
            float bmax = -INFINITY;
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                float v = s[e] * c;
                if (mask) {
                    const int key = BK * b + 32 * kq + 8 * (e >> 2) + 4 * half + (e & 3);
                    v = key <= qpos ? v : -INFINITY;
                }
                s[e] = v;
                bmax = fmaxf(bmax, v);
            }
            bmax = max_xor32(bmax);  // the other 32-lane half's keys of the same query rows
            const float mn = fmaxf(m, bmax);
            const float mr = mn == -INFINITY ? 0.f : mn;  // no key of this wave visible yet: nothing changes
            const float alpha = __builtin_amdgcn_exp2f(m - mr);
            m = mn;
            float bsum = 0.f;
            bf16x8_t pf[2];
#pragma unroll
            for (int u = 0; u < 2; ++u)
#pragma unroll
                for (int v = 0; v < 8; ++v) {
                    const float p = __builtin_amdgcn_exp2f(s[8 * u + v] - mr);
                    bsum += p;
                    pf[u][v] = (__bf16)p;
                }
            bsum = sum_xor32(bsum);
            l = l * alpha + bsum;
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int e = 0; e < 16; ++e) o[i][e] *= alpha;
            // O^T += V^T P^T: K step u covers keys 32 kq + 16 u + {4 half + 0..3, 8 + 4 half + 0..3}
#pragma unroll
            for (int u = 0; u < 2; ++u) {
                const int key = 32 * kq + 16 * u + 4 * half;
#pragma unroll
                for (int dt = 0; dt < 4; ++dt) {
                    const uint16_t* row = vt[32 * dt + ql];
                    const uint2 a0 = *reinterpret_cast<const uint2*>(row + vt_col(32 * dt, key));
                    const uint2 a1 = *reinterpret_cast<const uint2*>(row + vt_col(32 * dt, key + 8));
                    const uint4 av = make_uint4(a0.x, a0.y, a1.x, a1.y);
                    o[dt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, av), pf[u], o[dt],
                                                                    0, 0, 0);
                }
            }
        }
        if (b + 1 < nblk) {  // stage block b + 1 (its stage was last read for block b - 1)
            store_kv<KPT, VPAD>(kv, stage_k((b + 1) & 1), stage_v((b + 1) & 1), tid);
            if (b + 2 < nblk) load_kv<KPT>(kv, kc, vc, BK * (b + 2), last, tid);
        }
    }
    // KS waves per head: each finishes the d tiles dt with dt % KS == kq, from every wave's O^T,
    // max and sum handed over in LDS (a wave whose keys all lie after a query's position keeps
    // max -inf, sum 0 and O^T 0 for it)
    float f[KS], inv;
    {
        __syncthreads();  // every wave is done with the stages: they become the combine area
        float4* xo = reinterpret_cast<float4*>(smem);  // [HPW][dt][KS - 1 slots][e / 4][lane]
        float* ml = reinterpret_cast<float*>(smem + T::kXo);  // [HPW][KS][max, sum][lane]
        ml[((hw * KS + kq) * 2) * 64 + lane] = m;
        ml[((hw * KS + kq) * 2 + 1) * 64 + lane] = l;
#pragma unroll
        for (int dt = 0; dt < 4; ++dt) {
            const int own = dt % KS;
            if (own == kq) continue;
            const int slot = kq < own ? kq : kq - 1;
#pragma unroll
            for (int j = 0; j < 4; ++j)
                xo[(((hw * 4 + dt) * (KS - 1) + slot) * 4 + j) * 64 + lane] =
                    make_float4(o[dt][4 * j], o[dt][4 * j + 1], o[dt][4 * j + 2], o[dt][4 * j + 3]);
        }
        __syncthreads();
        float mx = -INFINITY;
#pragma unroll
        for (int j = 0; j < KS; ++j) {
            f[j] = ml[((hw * KS + j) * 2) * 64 + lane];
            mx = fmaxf(mx, f[j]);  // finite: key 0 lies in wave 0's part, visible to every query
        }
        float den = 0.f;
#pragma unroll
        for (int j = 0; j < KS; ++j) {
            f[j] = __builtin_amdgcn_exp2f(f[j] - mx);
            den += ml[((hw * KS + j) * 2 + 1) * 64 + lane] * f[j];
        }
        inv = 1.0f / den;
#pragma unroll
        for (int dt = 0; dt < 4; ++dt) {
            const int own = dt % KS;
            if (own != kq) continue;
#pragma unroll
            for (int j4 = 0; j4 < 4; ++j4) {
                float acc[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int j = 0; j < KS; ++j) {
                    float4 w;
                    if (j == kq) {
                        w = make_float4(o[dt][4 * j4], o[dt][4 * j4 + 1], o[dt][4 * j4 + 2], o[dt][4 * j4 + 3]);
                    } else {
                        const int slot = j < own ? j : j - 1;
                        w = xo[(((hw * 4 + dt) * (KS - 1) + slot) * 4 + j4) * 64 + lane];
                    }
                    acc[0] += w.x * f[j];
                    acc[1] += w.y * f[j];
                    acc[2] += w.z * f[j];
                    acc[3] += w.w * f[j];
                }
#pragma unroll
                for (int i = 0; i < 4; ++i) o[dt][4 * j4 + i] = acc[i];
            }
        }
    }
    if (t0 + ql >= n) return;
    uint16_t* orow = out + ((size_t)(t0 + ql) * kQH + qh) * kD;
    // O^T element e of d tile dt: d = 32 dt + 8 (e / 4) + 4 half + e % 4
#pragma unroll
    for (int dt = 0; dt < 4; ++dt) {
        if (dt % KS != kq) continue;
#pragma unroll
        for (int bq = 0; bq < 4; ++bq) {
            const int d = 32 * dt + 8 * bq + 4 * half;
            uint2 w;
            w.x = pack_bf16x2(o[dt][4 * bq] * inv, o[dt][4 * bq + 1] * inv);
            w.y = pack_bf16x2(o[dt][4 * bq + 2] * inv, o[dt][4 * bq + 3] * inv);
            *reinterpret_cast<uint2*>(orow + d) = w;
        }
    }
}

template <int HPW, int KS>
void launch_prefill(const void* q, const void* k_cache, const void* v_cache, const void* start, void* out, int n,
                    int L, hipStream_t stream) {
    const dim3 grid((unsigned)((n + kBQ - 1) / kBQ), (unsigned)(kKH * (4 / HPW)));
    hipLaunchKernelGGL((prefill_attention_kernel<HPW, KS>), grid, dim3(Tile<HPW, KS>::kThreads), 0, stream,
                       (const uint16_t*)q, (const uint16_t*)k_cache, (const uint16_t*)v_cache,
                       (const int64_t*)start, (uint16_t*)out, n, L);
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
    // one workgroup per CU while it fits (2 heads x 4 key parts per workgroup up to 512 tokens: 16
    // workgroups per 32 tokens), then 4 heads x 2 key parts.  Measured on MI355X at start 0 (and
    // after a cached prefix), against 4 heads x 2 parts: 128 / 256 / 512 tokens in 7.4 / 9.5 /
    // 14.1 us against 9.3 / 12.2 / 18.9, 128 after 1900 rows in 34 against 53; 1024 and 2048 tokens
    // in 31 / 106 us against 40 / 117 with 2 heads x 4 parts
    if (n <= 512)
        launch_prefill<2, 4>(q, k_cache, v_cache, start, out, n, L, (hipStream_t)stream);
    else
        launch_prefill<4, 2>(q, k_cache, v_cache, start, out, n, L, (hipStream_t)stream);
    return moss_launch_status();
}
