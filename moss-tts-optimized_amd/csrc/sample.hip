// Decode-step sampling: top-k / top-p (nucleus) sampling with temperature over bf16 logits, and the
// composition of the next 33 input ids (text token + 32 audio codes) with the delay pattern.
//
// sample_topk (src/moss_tts/_runtime/llm.py:10-19): temperature <= 0 gives argmax (first maximal
// index); otherwise the top_k largest of logits / temperature (fp32) in descending order (ties:
// lower index first), their softmax, the entries whose cumulative probability before them exceeds
// top_p removed, and one index drawn in proportion to the rest.
// Random numbers: Philox4x32-10 (Salmon, Moraes, Dror and Shaw, "Parallel random numbers: as easy
// as 1, 2, 3", SC 2011), counter = (position, row, salt), key = the 64-bit seed read from a device
// buffer, so a captured decode graph draws fresh numbers at every position, and for every seed the
// host writes into that buffer between replays, without host involvement in the graph.  The draw inverts the
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

__device__ __forceinline__ float key_value(unsigned long long k) {
    const uint32_t u = (uint32_t)(k >> 32);
    return __uint_as_float((u >> 31) ? (u ^ 0x80000000u) : ~u);
}

__device__ __forceinline__ int key_index(unsigned long long k) { return (int)(0xFFFFFFFFu - (uint32_t)k); }

__device__ __forceinline__ unsigned long long wave_max_u64(unsigned long long k) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
        const unsigned long long o = __shfl_xor(k, off, kWave);
        k = o > k ? o : k;
    }
    return k;
}

__device__ __forceinline__ unsigned long long readlane_u64(unsigned long long v, int l) {
    const uint32_t lo = __builtin_amdgcn_readlane((uint32_t)v, l);
    const uint32_t hi = __builtin_amdgcn_readlane((uint32_t)(v >> 32), l);
    return ((unsigned long long)hi << 32) | lo;
}

// Number of lanes whose key is larger than this lane's.
__device__ __forceinline__ int wave_rank(unsigned long long v) {
    int r = 0;
#pragma unroll
    for (int l = 0; l < kWave; ++l) r += readlane_u64(v, l) > v;
    return r;
}

// One set of rows sampled with one setting (the arguments of moss_sample_topk).
struct SampleRows {
    const uint16_t* __restrict__ logits;
    int stride, vocab;
    float temperature;
    int top_k;
    float top_p;
    uint32_t salt;
    int64_t* __restrict__ out;
};

// One wave per row; lane l holds logits l + 64 j as unique keys (value, then lower index first).
// Selection: T = the k-th largest of the 64 per-lane maxima; at least k keys are >= T, so the top k
// are among the keys >= T.  Those candidates are compacted into LDS; when at most 64 remain (the
// usual case: about 31 for k = 25 over 1024 values) each lane ranks one against the others,
// otherwise k rounds of wave argmax run over the candidates.
__device__ __forceinline__ void sample_row(const SampleRows& a, int row, const uint64_t* __restrict__ seed,
                                           const int64_t* __restrict__ position) {
    __shared__ unsigned long long cand[kWave * kMaxPerLane];
    __shared__ float val[kMaxTopK];
    __shared__ int idx[kMaxTopK];
    __shared__ float prob[kMaxTopK];
    const uint16_t* logits = a.logits;
    const int stride = a.stride, vocab = a.vocab, top_k = a.top_k;
    const float temperature = a.temperature, top_p = a.top_p;
    const uint32_t salt = a.salt;
    int64_t* out = a.out;
    const int lane = threadIdx.x;
    const uint16_t* lr = logits + (size_t)row * stride;
    const bool greedy = !(temperature > 0.f);
    const int k = greedy ? 1 : top_k;
    uint16_t raw[kMaxPerLane];
#pragma unroll
    for (int j = 0; j < kMaxPerLane; ++j) raw[j] = lr[min(lane + kWave * j, vocab - 1)];  // no branch around loads
    unsigned long long keys[kMaxPerLane];
    unsigned long long lane_max = 0;
#pragma unroll
    for (int j = 0; j < kMaxPerLane; ++j) {
        const int i = lane + kWave * j;
        // greedy: the raw logits (argmax is unchanged by a positive scale); else logits / T in fp32
        const float x = greedy ? bf16_bits(raw[j]) : bf16_bits(raw[j]) / temperature;
        keys[j] = i < vocab ? order_key(x, i) : 0ull;  // every valid key is nonzero
        lane_max = keys[j] > lane_max ? keys[j] : lane_max;
    }
    // k <= min(vocab, 64) lanes hold a nonzero maximum, all distinct, so rank k - 1 exists
    const int max_rank = wave_rank(lane_max);  // every lane takes part in the readlanes
    const unsigned long long at_k = __ballot(lane_max != 0 && max_rank == k - 1);
    const unsigned long long thresh = at_k ? readlane_u64(lane_max, __ffsll((long long)at_k) - 1) : 1ull;
    int count = 0;
#pragma unroll
    for (int j = 0; j < kMaxPerLane; ++j) count += keys[j] >= thresh;
    int incl = count;
#pragma unroll
    for (int off = 1; off < kWave; off <<= 1) {
        const int o = __shfl_up(incl, off, kWave);
        if (lane >= off) incl += o;
    }
    const int total = __shfl(incl, kWave - 1, kWave);
    int slot = incl - count;
#pragma unroll
    for (int j = 0; j < kMaxPerLane; ++j)
        if (keys[j] >= thresh) cand[slot++] = keys[j];
    __syncthreads();
    if (total <= kWave) {
        const unsigned long long mine = lane < total ? cand[lane] : 0ull;
        const int r = wave_rank(mine);
        if (mine != 0 && r < k) {
            val[r] = key_value(mine);
            idx[r] = key_index(mine);
        }
    } else {
        unsigned long long ck[kMaxPerLane];
#pragma unroll
        for (int t = 0; t < kMaxPerLane; ++t) {
            const int q = lane + kWave * t;
            ck[t] = q < total ? cand[q] : 0ull;
        }
        for (int r = 0; r < k; ++r) {
            unsigned long long best = 0;
#pragma unroll
            for (int t = 0; t < kMaxPerLane; ++t) best = ck[t] > best ? ck[t] : best;
            best = wave_max_u64(best);  // keys are unique: exactly one entry equals it
#pragma unroll
            for (int t = 0; t < kMaxPerLane; ++t) ck[t] = ck[t] == best ? 0ull : ck[t];
            if (lane == 0) {
                val[r] = key_value(best);
                idx[r] = key_index(best);
            }
        }
    }
    __syncthreads();
    if (greedy) {
        if (lane == 0) out[row] = idx[0];
        return;
    }
    // softmax over the k values (descending, so val[0] is the maximum), then the top-p cut
    if (lane < k) prob[lane] = expf(val[lane] - val[0]);
    __syncthreads();
    if (lane != 0) return;
    float sum = 0.f;
    for (int r = 0; r < k; ++r) sum += prob[r];
    float cum = 0.f, total_p = 0.f;
    for (int r = 0; r < k; ++r) {
        float q = prob[r] / sum;
        cum += q;
        if (cum - q > top_p) q = 0.f;
        prob[r] = q;
        total_p += q;
    }
    const int64_t pos = *position;
    const uint64_t sd = *seed;
    const uint2 key = make_uint2((uint32_t)sd, (uint32_t)(sd >> 32));
    const uint4 rnd = philox4x32_10(make_uint4((uint32_t)pos, (uint32_t)((uint64_t)pos >> 32), (uint32_t)row, salt), key);
    const float u = (float)(rnd.x >> 8) * (1.0f / 16777216.0f);
    const float target = u * total_p;
    float acc = 0.f;
    int pick = 0;
    for (int r = 0; r < k; ++r) {
        if (prob[r] > 0.f) pick = r;  // the last kept entry, should rounding leave target uncovered
        acc += prob[r];
        if (prob[r] > 0.f && acc > target) break;
    }
    out[row] = idx[pick];
}

__global__ __launch_bounds__(64) void sample_topk_rows(SampleRows a, const uint64_t* __restrict__ seed,
                                                       const int64_t* __restrict__ position) {
    sample_row(a, blockIdx.x, seed, position);
}

// Two sets in one launch: workgroups [0, rows_a) sample set a, the rest set b (row numbering, and
// with it the random stream, restarts at 0 for b), each exactly as sample_topk_rows would.
__global__ __launch_bounds__(64) void sample_topk_pair(SampleRows a, int rows_a, SampleRows b,
                                                       const uint64_t* __restrict__ seed,
                                                       const int64_t* __restrict__ position) {
    if ((int)blockIdx.x < rows_a) sample_row(a, blockIdx.x, seed, position);
    else sample_row(b, (int)blockIdx.x - rows_a, seed, position);
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

// One in-audio step of the host loop, on the device (src/moss_tts/_runtime/streaming.py:107-112;
// inside the first 32 steps after the audio start it is the advance kernel of
// src/moss_tts/_runtime/first_audio_graph.py:14-29): the next ids become the step's input ids
// (and row `step` of the history), the position advances by one, the audio length grows when the
// text token is the audio start, gen-slot or delay-slot id, and the delay counter starts at the
// first delay-slot token and then counts every step.  status = (text token, audio length, delay,
// position) after the update.
__global__ __launch_bounds__(64) void advance_step_kernel(const int64_t* __restrict__ next_ids,
                                                          int64_t* __restrict__ ids, int64_t* __restrict__ position,
                                                          int64_t* __restrict__ audio_length,
                                                          int64_t* __restrict__ delay_length,
                                                          int64_t* __restrict__ history, int64_t* __restrict__ status,
                                                          int step, int width, int64_t audio_start_id,
                                                          int64_t gen_slot_id, int64_t delay_slot_id) {
    const int i = threadIdx.x;
    if (i < width) {
        const int64_t v = next_ids[i];
        ids[i] = v;
        if (history) history[(size_t)step * width + i] = v;
    }
    if (i == 0) {
        const int64_t text = next_ids[0];
        const int64_t pos = *position + 1;
        int64_t len = *audio_length;
        if (text == audio_start_id || text == gen_slot_id || text == delay_slot_id) ++len;
        int64_t delay = *delay_length;
        if (delay < 0 && text == delay_slot_id) delay = 0;
        if (delay >= 0) ++delay;
        *position = pos;
        *audio_length = len;
        *delay_length = delay;
        if (status) {
            status[0] = text;
            status[1] = len;
            status[2] = delay;
            status[3] = pos;
        }
    }
}

}  // namespace
}  // namespace moss

using namespace moss;

static bool sample_args_ok(const void* logits, int rows, int stride, int vocab, float temperature, int top_k,
                           const void* out) {
    return logits && out && rows > 0 && vocab > 0 && vocab <= kWave * kMaxPerLane && stride >= vocab &&
           (!(temperature > 0.f) || (top_k >= 1 && top_k <= kMaxTopK && top_k <= vocab)) && MOSS_ALIGNED(logits, 2) &&
           MOSS_ALIGNED(out, 8);
}

MOSS_API int moss_sample_topk(const void* logits, int rows, int stride, int vocab, float temperature, int top_k,
                              float top_p, const void* seed, const void* position, int salt, void* out,
                              void* stream) {
    MOSS_CHECK_ARG(sample_args_ok(logits, rows, stride, vocab, temperature, top_k, out));
    MOSS_CHECK_ARG(seed && position && MOSS_ALIGNED(seed, 8) && MOSS_ALIGNED(position, 8));
    const SampleRows a{(const uint16_t*)logits, stride, vocab, temperature, top_k, top_p, (uint32_t)salt,
                       (int64_t*)out};
    hipLaunchKernelGGL(sample_topk_rows, dim3(rows), dim3(kWave), 0, (hipStream_t)stream, a, (const uint64_t*)seed,
                       (const int64_t*)position);
    return moss_launch_status();
}

MOSS_API int moss_sample_topk_pair(const void* logits_a, int rows_a, int stride_a, int vocab_a, float temperature_a,
                                   int top_k_a, float top_p_a, int salt_a, void* out_a, const void* logits_b,
                                   int rows_b, int stride_b, int vocab_b, float temperature_b, int top_k_b,
                                   float top_p_b, int salt_b, void* out_b, const void* seed, const void* position,
                                   void* stream) {
    MOSS_CHECK_ARG(sample_args_ok(logits_a, rows_a, stride_a, vocab_a, temperature_a, top_k_a, out_a));
    MOSS_CHECK_ARG(sample_args_ok(logits_b, rows_b, stride_b, vocab_b, temperature_b, top_k_b, out_b));
    MOSS_CHECK_ARG(seed && position && MOSS_ALIGNED(seed, 8) && MOSS_ALIGNED(position, 8));
    const SampleRows a{(const uint16_t*)logits_a, stride_a, vocab_a, temperature_a, top_k_a, top_p_a,
                       (uint32_t)salt_a, (int64_t*)out_a};
    const SampleRows b{(const uint16_t*)logits_b, stride_b, vocab_b, temperature_b, top_k_b, top_p_b,
                       (uint32_t)salt_b, (int64_t*)out_b};
    hipLaunchKernelGGL(sample_topk_pair, dim3(rows_a + rows_b), dim3(kWave), 0, (hipStream_t)stream, a, rows_a, b,
                       (const uint64_t*)seed, (const int64_t*)position);
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

MOSS_API int moss_advance_step(const void* next_ids, void* ids, void* position, void* audio_length, void* delay_length,
                               void* history, void* status, int step, int width, long long audio_start_id,
                               long long gen_slot_id, long long delay_slot_id, void* stream) {
    MOSS_CHECK_ARG(next_ids && ids && position && audio_length && delay_length);
    MOSS_CHECK_ARG(width > 0 && width <= kWave && step >= 0);
    MOSS_CHECK_ARG(next_ids != ids);
    hipLaunchKernelGGL(advance_step_kernel, dim3(1), dim3(kWave), 0, (hipStream_t)stream, (const int64_t*)next_ids,
                       (int64_t*)ids, (int64_t*)position, (int64_t*)audio_length, (int64_t*)delay_length,
                       (int64_t*)history, (int64_t*)status, step, width, (int64_t)audio_start_id,
                       (int64_t)gen_slot_id, (int64_t)delay_slot_id);
    return moss_launch_status();
}
