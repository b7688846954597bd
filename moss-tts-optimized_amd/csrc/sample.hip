// Decode-step sampling: top-k / top-p (nucleus) sampling with temperature over bf16 logits, and the
// composition of the next 33 input ids (text token + 32 audio codes) with the delay pattern.
//
// sample_topk (src/moss_tts/_runtime/llm.py:10-19): temperature <= 0 gives argmax (first maximal
// index); otherwise the top_k largest of logits / temperature (fp32) in descending order (ties:
// lower index first), their softmax, the entries whose cumulative probability before them exceeds
// top_p removed, and one index drawn in proportion to the rest.
// Random numbers: Philox4x32-10 (Salmon, Moraes, Dror and Shaw, "Parallel random numbers: as easy
// as 1, 2, 3", SC 2011), counter = (position, row, salt), key = seed, so a captured decode graph
// draws fresh numbers at every position without host involvement.  The draw inverts the
// cumulative distribution: the first j with sum_{i <= j} p_i > u * sum_i p_i, u in [0, 1).
//
// compose_next_ids (src/moss_tts/_runtime/llm.py:280-287): text token = text_ids[text index],
// replaced by the delay-slot id while delay_length >= 0 and by the audio-end id at delay_length
// == 32; audio code c is kept when c < audio_length and (delay_length < 0 or c >= delay_length),
// else the pad code.
#include "common.h"

namespace moss {
namespace {

constexpr int kMaxTopK = 64;
constexpr int kMaxPerLane = 32;  // vocab <= 2048

__device__ __forceinline__ uint4 philox_round(uint4 c, uint2 k) {
    const uint32_t lo0 = 0xD2511F53u * c.x, hi0 = __umulhi(0xD2511F53u, c.x);
    const uint32_t lo1 = 0xCD9E8D57u * c.z, hi1 = __umulhi(0xCD9E8D57u, c.z);
    return make_uint4(hi1 ^ c.y ^ k.x, lo1, hi0 ^ c.w ^ k.y, lo0);
}

__device__ __forceinline__ uint4 philox4x32_10(uint4 c, uint2 k) {
#pragma unroll
    for (int r = 0; r < 10; ++r) {
        if (r > 0) k = make_uint2(k.x + 0x9E3779B9u, k.y + 0xBB67AE85u);
        c = philox_round(c, k);
    }
    return c;
}

// Total order on (value, index): larger value first, then lower index.
__device__ __forceinline__ unsigned long long order_key(float v, int i) {
    uint32_t u = __float_as_uint(v);
    u ^= (u >> 31) ? 0xFFFFFFFFu : 0x80000000u;
    return ((unsigned long long)u << 32) | (uint32_t)(0xFFFFFFFFu - (uint32_t)i);
}

__device__ __forceinline__ unsigned long long wave_max_u64(unsigned long long k) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
        const unsigned long long o = __shfl_xor(k, off, kWave);
        k = o > k ? o : k;
    }
    return k;
}

// One wave per row; lane l holds logits l + 64 j.
__global__ __launch_bounds__(64) void sample_topk_rows(const uint16_t* __restrict__ logits, int stride, int vocab,
                                                       float temperature, int top_k, float top_p, uint2 key,
                                                       const int64_t* __restrict__ position, uint32_t salt,
                                                       int64_t* __restrict__ out) {
    __shared__ float val[kMaxTopK];
    __shared__ int idx[kMaxTopK];
    __shared__ float prob[kMaxTopK];
    const int row = blockIdx.x, lane = threadIdx.x;
    const uint16_t* lr = logits + (size_t)row * stride;
    const bool greedy = !(temperature > 0.f);
    float v[kMaxPerLane];
#pragma unroll
    for (int j = 0; j < kMaxPerLane; ++j) {
        const int i = lane + kWave * j;
        // greedy: the raw logits (argmax is unchanged by a positive scale); else logits / T in fp32
        v[j] = i < vocab ? (greedy ? bf16_bits(lr[i]) : bf16_bits(lr[i]) / temperature) : -__builtin_inff();
    }
    const int k = greedy ? 1 : top_k;
    uint32_t taken = 0;
    for (int r = 0; r < k; ++r) {
        unsigned long long best = 0;
#pragma unroll
        for (int j = 0; j < kMaxPerLane; ++j) {
            const int i = lane + kWave * j;
            if (i < vocab && !((taken >> j) & 1u)) {
                const unsigned long long kk = order_key(v[j], i);
                best = kk > best ? kk : best;
            }
        }
        best = wave_max_u64(best);  // every lane holds the winner
        const int bi = (int)(0xFFFFFFFFu - (uint32_t)(best & 0xFFFFFFFFull));
        if ((bi & (kWave - 1)) == lane) {  // the owning lane marks it and publishes it
            float sel = 0.f;
#pragma unroll
            for (int j = 0; j < kMaxPerLane; ++j)
                if (j == bi / kWave) sel = v[j];
            taken |= 1u << (bi / kWave);
            val[r] = sel;
            idx[r] = bi;
        }
    }
    __syncthreads();
    if (lane != 0) return;
    if (greedy) {
        out[row] = idx[0];
        return;
    }
    // softmax over the k values (descending, so val[0] is the maximum), then the top-p cut
    float sum = 0.f;
    for (int r = 0; r < k; ++r) {
        prob[r] = expf(val[r] - val[0]);
        sum += prob[r];
    }
    float cum = 0.f, total = 0.f;
    for (int r = 0; r < k; ++r) {
        float q = prob[r] / sum;
        cum += q;
        if (cum - q > top_p) q = 0.f;
        prob[r] = q;
        total += q;
    }
    const int64_t pos = *position;
    const uint4 rnd = philox4x32_10(make_uint4((uint32_t)pos, (uint32_t)((uint64_t)pos >> 32), (uint32_t)row, salt), key);
    const float u = (float)(rnd.x >> 8) * (1.0f / 16777216.0f);
    const float target = u * total;
    float acc = 0.f;
    int pick = 0;
    for (int r = 0; r < k; ++r) {
        if (prob[r] > 0.f) pick = r;  // the last kept entry, should rounding leave target uncovered
        acc += prob[r];
        if (prob[r] > 0.f && acc > target) break;
    }
    out[row] = idx[pick];
}

__global__ __launch_bounds__(64) void compose_next_ids_kernel(const int64_t* __restrict__ text_index,
                                                              const int64_t* __restrict__ audio_index,
                                                              const int64_t* __restrict__ text_ids,
                                                              const int64_t* __restrict__ audio_length,
                                                              const int64_t* __restrict__ delay_length,
                                                              int64_t delay_slot_id, int64_t audio_end_id,
                                                              int channels, int64_t pad_code,
                                                              int64_t* __restrict__ next_ids) {
    const int c = threadIdx.x;
    const int64_t delay = *delay_length;
    if (c == 0) {
        const int64_t t = *text_index;
        int64_t tok = text_ids[t < 0 ? 0 : (t > 1 ? 1 : t)];
        if (delay >= 0) tok = delay_slot_id;
        if (delay == 32) tok = audio_end_id;
        next_ids[0] = tok;
    }
    if (c < channels) {
        const bool valid = (int64_t)c < *audio_length && (delay < 0 || (int64_t)c >= delay);
        next_ids[1 + c] = valid ? audio_index[c] : pad_code;
    }
}

}  // namespace
}  // namespace moss

using namespace moss;

MOSS_API int moss_sample_topk(const void* logits, int rows, int stride, int vocab, float temperature, int top_k,
                              float top_p, unsigned long long seed, const void* position, int salt, void* out,
                              void* stream) {
    MOSS_CHECK_ARG(logits && position && out && rows > 0 && vocab > 0 && vocab <= kWave * kMaxPerLane &&
                   stride >= vocab);
    MOSS_CHECK_ARG(!(temperature > 0.f) || (top_k >= 1 && top_k <= kMaxTopK && top_k <= vocab));
    MOSS_CHECK_ARG(MOSS_ALIGNED(logits, 2) && MOSS_ALIGNED(position, 8) && MOSS_ALIGNED(out, 8));
    const uint2 key = make_uint2((uint32_t)seed, (uint32_t)(seed >> 32));
    hipLaunchKernelGGL(sample_topk_rows, dim3(rows), dim3(kWave), 0, (hipStream_t)stream, (const uint16_t*)logits,
                       stride, vocab, temperature, top_k, top_p, key, (const int64_t*)position, (uint32_t)salt,
                       (int64_t*)out);
    return moss_launch_status();
}

MOSS_API int moss_compose_next_ids(const void* text_index, const void* audio_index, const void* text_ids,
                                   const void* audio_length, const void* delay_length, long long delay_slot_id,
                                   long long audio_end_id, int channels, long long pad_code, void* next_ids,
                                   void* stream) {
    MOSS_CHECK_ARG(text_index && audio_index && text_ids && audio_length && delay_length && next_ids);
    MOSS_CHECK_ARG(channels > 0 && channels <= kWave);
    hipLaunchKernelGGL(compose_next_ids_kernel, dim3(1), dim3(kWave), 0, (hipStream_t)stream,
                       (const int64_t*)text_index, (const int64_t*)audio_index, (const int64_t*)text_ids,
                       (const int64_t*)audio_length, (const int64_t*)delay_length, (int64_t)delay_slot_id,
                       (int64_t)audio_end_id, channels, (int64_t)pad_code, (int64_t*)next_ids);
    return moss_launch_status();
}
