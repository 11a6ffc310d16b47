// stream_probe.hip -- single-launch HBM streaming ceiling on gfx950 (measurement only).
//
// One kernel that only streams: every wave reads one contiguous chunk of the
// buffer (L loads per lane, all issued before the first use, like the GEMV's
// weight loads), folds what it read with XOR and writes ONE word per wave. It
// bounds what any kernel reading the same bytes in one dispatch can reach on
// this GPU, ramp-up and drain included. bench.py --stream-ceiling drives it.
//
// Memory safety is decided on the host before any launch: the kernel reads
// exactly waves * chunk bytes from the start of the buffer (chunk = 64 lanes x
// L loads x load width) and writes exactly `waves` words of `out`; the entry
// point refuses a call whose buffer or output is smaller than that.

#include <hip/hip_runtime.h>

#include <stdint.h>
#include <stdio.h>

namespace {

thread_local char g_probe_error[256] = "";

template <typename V>
__device__ __forceinline__ uint32_t fold(V v);
template <>
__device__ __forceinline__ uint32_t fold<uint32_t>(uint32_t v) {
    return v;
}
template <>
__device__ __forceinline__ uint32_t fold<uint4>(uint4 v) {
    return v.x ^ v.y ^ v.z ^ v.w;
}

// Wave w reads elements [w * L * 64, (w + 1) * L * 64) of V: load i of lane l
// is element w * L * 64 + i * 64 + l, so every load instruction of a wave is
// one contiguous, fully coalesced run.
template <typename V, int L>
__global__ __launch_bounds__(512) void stream_read_kernel(const V *__restrict__ src, uint32_t *__restrict__ out,
                                                          int64_t waves) {
    const int64_t wave = static_cast<int64_t>(blockIdx.x) * (blockDim.x >> 6) + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (wave >= waves) return;
    const V *p = src + wave * (L * 64) + lane;
    V v[L];
#pragma unroll
    for (int i = 0; i < L; ++i) v[i] = p[i * 64];
    uint32_t s = 0;
#pragma unroll
    for (int i = 0; i < L; ++i) s ^= fold<V>(v[i]);
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) s ^= __shfl_xor(s, off, 64);
    if (lane == 0) out[wave] = s;
}

template <typename V, int L>
void launch(const void *buf, uint32_t *out, int64_t waves, int threads, hipStream_t stream) {
    const int64_t per_wg = threads / 64;
    const unsigned grid = static_cast<unsigned>((waves + per_wg - 1) / per_wg);
    hipLaunchKernelGGL((stream_read_kernel<V, L>), dim3(grid), dim3(threads), 0, stream,
                       static_cast<const V *>(buf), out, waves);
}

}  // namespace

extern "C" {

const char *ternel_probe_last_error(void) { return g_probe_error; }

// Bytes one wave reads for a (width, loads) pair; 0 if unsupported.
int64_t ternel_probe_chunk_bytes(int width, int loads) {
    if ((width != 4 && width != 16) || (loads != 1 && loads != 2 && loads != 4 && loads != 7 && loads != 8 &&
                                        loads != 16 && loads != 28))
        return 0;
    return static_cast<int64_t>(width) * 64 * loads;
}

// Streams the first `waves * chunk` bytes of buf (chunk from
// ternel_probe_chunk_bytes) with `threads`-thread workgroups and writes one
// word per wave to out. Returns 0, or -1 with a message when the call would
// read past `buf_bytes` or write past `out_words`.
int ternel_probe_stream(const void *buf, int64_t buf_bytes, uint32_t *out, int64_t out_words, int64_t waves,
                        int width, int loads, int threads, void *stream) {
    g_probe_error[0] = '\0';
    const int64_t chunk = ternel_probe_chunk_bytes(width, loads);
    if (chunk == 0) {
        snprintf(g_probe_error, sizeof(g_probe_error), "unsupported width %d / loads %d", width, loads);
        return -1;
    }
    if (threads != 256 && threads != 512) {
        snprintf(g_probe_error, sizeof(g_probe_error), "threads must be 256 or 512, got %d", threads);
        return -1;
    }
    if (!buf || !out || waves <= 0 || waves > buf_bytes / chunk || waves > out_words) {
        snprintf(g_probe_error, sizeof(g_probe_error),
                 "%lld waves of %lld bytes do not fit a %lld-byte buffer and %lld output words",
                 static_cast<long long>(waves), static_cast<long long>(chunk), static_cast<long long>(buf_bytes),
                 static_cast<long long>(out_words));
        return -1;
    }
    if (reinterpret_cast<uintptr_t>(buf) % 16) {
        snprintf(g_probe_error, sizeof(g_probe_error), "buffer must be 16-byte aligned");
        return -1;
    }
    hipStream_t s = static_cast<hipStream_t>(stream);
#define PROBE_CASE(W, V, LL)                                    \
    if (width == W && loads == LL) launch<V, LL>(buf, out, waves, threads, s);
    PROBE_CASE(4, uint32_t, 1)
    PROBE_CASE(4, uint32_t, 2)
    PROBE_CASE(4, uint32_t, 4)
    PROBE_CASE(4, uint32_t, 7)
    PROBE_CASE(4, uint32_t, 8)
    PROBE_CASE(4, uint32_t, 16)
    PROBE_CASE(4, uint32_t, 28)
    PROBE_CASE(16, uint4, 1)
    PROBE_CASE(16, uint4, 2)
    PROBE_CASE(16, uint4, 4)
    PROBE_CASE(16, uint4, 7)
    PROBE_CASE(16, uint4, 8)
    PROBE_CASE(16, uint4, 16)
    PROBE_CASE(16, uint4, 28)
#undef PROBE_CASE
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) {
        snprintf(g_probe_error, sizeof(g_probe_error), "launch failed: %s", hipGetErrorString(e));
        return -2;
    }
    return 0;
}

}  // extern "C"
