// Streaming read of a byte range: the measurement kernel that bench.py times on the bytes of a
// decode GEMV, so the ceiling of one launch that only reads those bytes is measured beside the
// GEMV (a launch of this size spends a fixed ~1.7 us before any byte moves).  No counterpart in
// the reference.
//
// Each 256-thread workgroup covers 16 KiB: load u of thread t reads 16-byte chunk
// 1024 b + 256 u + t, so every wave instruction reads 1 KiB contiguous; all four loads are issued
// before any is used.  Each wave XOR-reduces its words (order-free, so the result is
// deterministic) with DPP moves and lane reads, no LDS and no barrier, and stores one word,
// xor_out[4 b + w], which keeps every load live.  (Measured on MI355X for 29 MB: a workgroup
// reduction through LDS and a barrier cost ~0.4 us per launch more, nontemporal stores ~3 us.)
#include "common.h"

namespace moss {
namespace {

constexpr int kChunksPerThread = 4;
constexpr long long kBytesPerWorkgroup = 256LL * 16 * kChunksPerThread;

typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));

template <int CTRL>
__device__ __forceinline__ uint32_t dpp_u32(uint32_t v) {
    return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, CTRL, 0xf, 0xf, false);
}

__global__ __launch_bounds__(256) void stream_read_xor(const u32x4_t* __restrict__ src, long long n16,
                                                       uint32_t* __restrict__ xor_out) {
    const long long base = (long long)blockIdx.x * 256 * kChunksPerThread + threadIdx.x;
    u32x4_t v[kChunksPerThread];
#pragma unroll
    for (int u = 0; u < kChunksPerThread; ++u) {
        const long long i = base + 256LL * u;
        v[u] = i < n16 ? __builtin_nontemporal_load(src + i) : u32x4_t{0u, 0u, 0u, 0u};
    }
    uint32_t a = 0u;
#pragma unroll
    for (int u = 0; u < kChunksPerThread; ++u) a ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
    a ^= dpp_u32<0xB1>(a);   // quad_perm [1,0,3,2]
    a ^= dpp_u32<0x4E>(a);   // quad_perm [2,3,0,1]
    a ^= dpp_u32<0x141>(a);  // row_half_mirror
    a ^= dpp_u32<0x140>(a);  // row_mirror: every lane holds its 16-lane row's XOR
    a = (uint32_t)(__builtin_amdgcn_readlane((int)a, 0) ^ __builtin_amdgcn_readlane((int)a, 16) ^
                   __builtin_amdgcn_readlane((int)a, 32) ^ __builtin_amdgcn_readlane((int)a, 48));
    if ((threadIdx.x & (kWave - 1)) == 0) xor_out[4LL * blockIdx.x + threadIdx.x / kWave] = a;
}

}  // namespace
}  // namespace moss

using namespace moss;

static long long stream_read_workgroups(long long bytes) {
    return bytes > 0 ? (bytes + kBytesPerWorkgroup - 1) / kBytesPerWorkgroup : 0;
}

MOSS_API long long moss_stream_read_words(long long bytes) { return 4 * stream_read_workgroups(bytes); }

MOSS_API int moss_stream_read(const void* src, long long bytes, void* xor_out, void* stream) {
    MOSS_CHECK_ARG(src && xor_out && bytes > 0 && bytes % 16 == 0 && MOSS_ALIGNED(src, 16) && MOSS_ALIGNED(xor_out, 4));
    const long long wgs = stream_read_workgroups(bytes);
    MOSS_CHECK_ARG(wgs <= 0x7fffffffLL);
    hipLaunchKernelGGL(stream_read_xor, dim3((unsigned)wgs), dim3(256), 0, (hipStream_t)stream,
                       (const u32x4_t*)src, bytes / 16, (uint32_t*)xor_out);
    return moss_launch_status();
}
