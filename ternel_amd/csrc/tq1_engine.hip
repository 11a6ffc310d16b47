// tq1_engine.hip -- TQ1_G128 packed-weight kernels for MI355X (gfx950, CDNA4).
//
// One shared library, C ABI only (include/ternel_tq1.h).
//
// Device layout ("packed"): the canonical 28-byte blocks, permuted at 4-byte
// granularity into 64-row tiles -- word j (bytes 4j..4j+3) of block (row r,
// group g) lives at packed[((r / 64) * G + g) * 7 + j][r % 64]. A wave64 whose
// lanes own 64 consecutive rows therefore reads one word of one group with a
// single fully coalesced 256-byte load, and a tile of rows for one group is one
// contiguous 1,792-byte run. Rows past the end of the last tile are zero words.
// The permutation is exact in both directions (interleave_kernel /
// deinterleave_kernel); nothing is re-encoded, the weight stays 28 bytes per
// 128 weights.
//
// Kernels:
//   validate_kernel    fail-closed byte scan of canonical blocks
//   decode_kernel      bit-exact trit decode of canonical blocks (test entry)
//   interleave_kernel / deinterleave_kernel   canonical <-> packed
//   lut_gemv_kernel    LUT23 product, M = 1 decode GEMV and small batches,
//                      with a fused, ordered split-K fix-up
//   mfma_gemm_kernel   trits -> fp16 LDS tiles -> v_mfma_f32_32x32x16_f16
//   get_rows_kernel    packed embedding-row gather

#include <hip/hip_runtime.h>

#include <stdarg.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <algorithm>
#include <atomic>
#include <mutex>
#include <set>
#include <string>
#include <utility>
#include <type_traits>

#include "ternel_tq1.h"
#include "tq1_bytes.h"

namespace {

// Format constants (src/bonsai_tq1/format.py:14-24, lut23_reorder.py:27-29).
constexpr int kBlockWeights = 128;
constexpr int kBlockBytes = 28;
constexpr int kBlockWords = 7;
constexpr int kCodeSlots = 26;
using tq1_bytes::kFullSlots;
using tq1_bytes::kMaxTailByte;

// Packed layout: 64-row tiles, 7 words per block.
constexpr int kTileRows = 64;
constexpr int kTileGroupWords = kBlockWords * kTileRows;  // 448 words per (tile, group)

// LUT23 tables of one 128-weight group (geometry in tq1_bytes.h).
using tq1_bytes::kL2Entries;
using tq1_bytes::kL3Entries;
using tq1_bytes::kL3Base;
using tq1_bytes::kTailBase;
using tq1_bytes::kLutFloats;
// The kernels lay a set of tables out in two regions (three-trit, then
// two-trit): these are one group's share of each.
constexpr int kLut3Floats = (tq1_bytes::kFullSlots + 1) * kL3Entries;  // 702: 25 slots and the tail
constexpr int kLut2Floats = tq1_bytes::kFullSlots * kL2Entries;        // 225
static_assert(kLut3Floats + kLut2Floats == kLutFloats, "the regions hold a group's 927 floats");

constexpr int kThreads = 256;

// Split workspaces start with 64 KiB of 32-bit counters; the last one is the
// error word (the host section keeps every kernel's counters below it).
constexpr int kWorkspaceCounterBytes = 64 * 1024;
constexpr int kWorkspaceErrorSlot = kWorkspaceCounterBytes / 4 - 1;

// Phase timestamps (built only with -DTERNEL_TQ1_PROFILE, into a separate
// library that bench.py --phase-profile loads): lane 0 of each wave of the
// M = 1 stream GEMV writes the 100 MHz wall clock at its phase boundaries.
constexpr int kPhaseWaves = 8192;
constexpr int kPhaseSlots = 16;
#ifdef TERNEL_TQ1_PROFILE
__device__ unsigned long long g_phase_stamps[kPhaseWaves][kPhaseSlots];
#define TQ1_PHASE(wave_id, slot)                                                                     \
    do {                                                                                             \
        __builtin_amdgcn_sched_barrier(0);                                                           \
        if ((threadIdx.x & 63) == 0 && (wave_id) < kPhaseWaves)                                      \
            g_phase_stamps[(wave_id)][(slot)] = static_cast<unsigned long long>(wall_clock64());      \
        __builtin_amdgcn_sched_barrier(0);                                                           \
    } while (0)
// The last slot holds 1 + the XCC the wave runs on (wall clocks of waves on
// different XCCs are not comparable).
#define TQ1_PHASE_XCC(wave_id)                                                                       \
    do {                                                                                             \
        unsigned xcc;                                                                                \
        asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(xcc));                           \
        if ((threadIdx.x & 63) == 0 && (wave_id) < kPhaseWaves)                                      \
            g_phase_stamps[(wave_id)][kPhaseSlots - 1] = 1ull + (xcc & 0xfu);                        \
    } while (0)
#else
#define TQ1_PHASE_XCC(wave_id) \
    do {                       \
    } while (0)
#define TQ1_PHASE(wave_id, slot) \
    do {                         \
    } while (0)
#endif

thread_local char g_last_error[512] = "";

int fail(int code, const char *fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
    va_end(ap);
    return code;
}

#define TQ1_LAUNCH_CHECK()                                                                    \
    do {                                                                                      \
        hipError_t err_ = hipGetLastError();                                                  \
        if (err_ != hipSuccess)                                                               \
            return fail(TERNEL_TQ1_EHIP, "kernel launch failed: %s", hipGetErrorString(err_)); \
    } while (0)

// ---------------------------------------------------------------------------
// Scalar conversions. fp16 via _Float16 (v_cvt_f32_f16 keeps subnormals, inf
// and NaN); bf16 by bit manipulation with round-to-nearest-even.
// ---------------------------------------------------------------------------
struct bf16_t {
    uint16_t bits;
};

__device__ __forceinline__ float half_bits_to_float(uint32_t bits) {
    const uint16_t b = static_cast<uint16_t>(bits);
    _Float16 h;
    __builtin_memcpy(&h, &b, sizeof(h));
    return static_cast<float>(h);
}

template <typename T>
__device__ __forceinline__ float to_f32(T v);
template <>
__device__ __forceinline__ float to_f32<_Float16>(_Float16 v) {
    return static_cast<float>(v);
}
template <>
__device__ __forceinline__ float to_f32<bf16_t>(bf16_t v) {
    return __uint_as_float(static_cast<uint32_t>(v.bits) << 16);
}
template <>
__device__ __forceinline__ float to_f32<float>(float v) {
    return v;
}

template <typename T>
__device__ __forceinline__ T from_f32(float v);
template <>
__device__ __forceinline__ _Float16 from_f32<_Float16>(float v) {
    return static_cast<_Float16>(v);
}
template <>
__device__ __forceinline__ bf16_t from_f32<bf16_t>(float v) {
    uint32_t u = __float_as_uint(v);
    bf16_t out;
    if ((u & 0x7fffffffu) > 0x7f800000u) {
        out.bits = static_cast<uint16_t>((u >> 16) | 0x0040u);  // quiet NaN, sign kept
    } else {
        u += 0x7fffu + ((u >> 16) & 1u);
        out.bits = static_cast<uint16_t>(u >> 16);
    }
    return out;
}
template <>
__device__ __forceinline__ float from_f32<float>(float v) {
    return v;
}

__device__ __forceinline__ uint32_t block_byte(const uint32_t (&w)[kBlockWords], int index) {
    return (w[index >> 2] >> ((index & 3) * 8)) & 0xffu;
}

__device__ __forceinline__ uint32_t wave_sum_u32(uint32_t v) {
#pragma unroll
    for (int offset = 32; offset > 0; offset >>= 1) v += __shfl_xor(v, offset, 64);
    return v;
}

__device__ __forceinline__ int64_t packed_word_index(int64_t row, int64_t G, int64_t g, int j) {
    return (((row / kTileRows) * G + g) * kBlockWords + j) * kTileRows + (row % kTileRows);
}

// ---------------------------------------------------------------------------
// Helpers
// ---------------------------------------------------------------------------
__device__ __forceinline__ int ceil_div_dev(int a, int b) { return (a + b - 1) / b; }

__global__ void zero_u64_kernel(unsigned long long *p, int n) {
    const int i = threadIdx.x;
    if (i < n) p[i] = 0ull;
}

// ---------------------------------------------------------------------------
// validate_kernel: counts regular code bytes > 242 and tail bytes > 26 in
// canonical blocks, walked as 32-bit words; word j (0..6) of a block holds
//   j = 0: scale, scale, code0, code1      j = 1..5: four codes
//   j = 6: code22, code23, code24, tail.
// SWAR per byte b:  b >= 243  <=>  bit7(b) & bit7((b & 0x7f) + 13)
//                   b >= 27   <=>  bit7(b) | bit7((b & 0x7f) + 101)
// (the additions never carry across bytes).
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(kThreads) void validate_kernel(const uint32_t *__restrict__ words,
                                                            int64_t nwords,
                                                            unsigned long long *counters) {
    const int64_t first = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
    int j = static_cast<int>(first % kBlockWords);
    const int step = static_cast<int>(stride % kBlockWords);
    uint32_t bad_regular = 0, bad_tail = 0;
    for (int64_t w = first; w < nwords; w += stride) {
        const uint32_t d = words[w];
        const uint32_t regular_mask = j == 0 ? 0x80800000u : (j == 6 ? 0x00808080u : 0x80808080u);
        const uint32_t tail_mask = j == 6 ? 0x80000000u : 0u;
        const uint32_t low7 = d & 0x7f7f7f7fu;
        bad_regular += __popc(d & (low7 + 0x0d0d0d0du) & regular_mask);
        bad_tail += __popc((d | (low7 + 0x65656565u)) & tail_mask);
        j += step;
        if (j >= kBlockWords) j -= kBlockWords;
    }
    bad_regular = wave_sum_u32(bad_regular);
    bad_tail = wave_sum_u32(bad_tail);
    if ((threadIdx.x & 63) == 0) {
        if (bad_regular) atomicAdd(&counters[0], static_cast<unsigned long long>(bad_regular));
        if (bad_tail) atomicAdd(&counters[1], static_cast<unsigned long long>(bad_tail));
    }
}

// ---------------------------------------------------------------------------
// decode_kernel: one thread per (block, code slot); trit i of a byte is
// (b / 3^i) % 3, exactly as src/bonsai_tq1/format.py:112-121 computes it.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(kThreads) void decode_kernel(const uint8_t *__restrict__ blocks,
                                                          int64_t nblocks,
                                                          uint8_t *__restrict__ scales_out,
                                                          uint8_t *__restrict__ codes_out) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i >= nblocks * kCodeSlots) return;
    const int64_t n = i / kCodeSlots;
    const int s = static_cast<int>(i - n * kCodeSlots);
    const uint8_t *blk = blocks + n * kBlockBytes;
    const uint32_t b = blk[2 + s];
    uint8_t *codes = codes_out + n * kBlockWeights;
    if (s < kFullSlots) {
        codes[5 * s + 0] = static_cast<uint8_t>(b % 3u);
        codes[5 * s + 1] = static_cast<uint8_t>((b / 3u) % 3u);
        codes[5 * s + 2] = static_cast<uint8_t>((b / 9u) % 3u);
        codes[5 * s + 3] = static_cast<uint8_t>((b / 27u) % 3u);
        codes[5 * s + 4] = static_cast<uint8_t>((b / 81u) % 3u);
    } else {
        codes[125] = static_cast<uint8_t>(b % 3u);
        codes[126] = static_cast<uint8_t>((b / 3u) % 3u);
        codes[127] = static_cast<uint8_t>((b / 9u) % 3u);
        scales_out[n * 2 + 0] = blk[0];
        scales_out[n * 2 + 1] = blk[1];
    }
}

// ---------------------------------------------------------------------------
// q2_to_tq1_kernel: Q2_0/g128 blocks (34 bytes: fp16 scale, 32 bytes of 2-bit
// codes, code c in bits 2(c%4).. of byte 2 + c/4) re-encoded as TQ1_G128 blocks
// on the device -- decode_q2_blocks then encode_tq1_blocks of
// src/bonsai_tq1/format.py:51-91 in one pass. One thread per (block, output
// slot): slot 0 copies the scale, slots 1..25 pack codes 5(s-1).. as base-3
// bytes, slot 26 the tail codes 125..127. Codes of value 3 have no ternary
// meaning; they are counted (the caller rejects the source) and the byte is
// written as if they were 2.
// ---------------------------------------------------------------------------
constexpr int kQ2BlockBytes = 34;
constexpr int kQ2Slots = 27;  // the scale pair, 25 regular bytes, the tail byte

__global__ __launch_bounds__(kThreads) void q2_to_tq1_kernel(const uint8_t *__restrict__ q2, uint8_t *__restrict__ tq1,
                                                             int64_t nblocks, unsigned long long *bad_codes) {
    const int64_t total = nblocks * kQ2Slots;
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < total;
         i += static_cast<int64_t>(gridDim.x) * blockDim.x) {
        const int64_t n = i / kQ2Slots;
        const int slot = static_cast<int>(i - n * kQ2Slots);
        const uint8_t *src = q2 + n * kQ2BlockBytes;
        uint8_t *dst = tq1 + n * kBlockBytes;
        if (slot == 0) {
            dst[0] = src[0];
            dst[1] = src[1];
            continue;
        }
        const int first = slot <= kFullSlots ? 5 * (slot - 1) : 125;
        const int count = slot <= kFullSlots ? 5 : 3;
        unsigned value = 0, power = 1, bad = 0;
        for (int k = 0; k < count; ++k) {
            const int c = first + k;
            unsigned code = (src[2 + (c >> 2)] >> ((c & 3) * 2)) & 3u;
            bad += code == 3u;
            code = code == 3u ? 2u : code;
            value += code * power;
            power *= 3u;
        }
        dst[slot + 1] = static_cast<uint8_t>(value);
        if (bad) atomicAdd(bad_codes, static_cast<unsigned long long>(bad));
    }
}

// ---------------------------------------------------------------------------
// interleave_kernel / deinterleave_kernel: canonical blocks <-> packed words.
// One thread per packed word (writes coalesced) / per canonical word.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(kThreads) void interleave_kernel(const uint32_t *__restrict__ canonical,
                                                              uint32_t *__restrict__ packed, int64_t rows,
                                                              int64_t G, int64_t total_words) {
    const int64_t w = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (w >= total_words) return;
    const int lane = static_cast<int>(w % kTileRows);
    const int64_t rest = w / kTileRows;
    const int j = static_cast<int>(rest % kBlockWords);
    const int64_t tg = rest / kBlockWords;
    const int64_t g = tg % G;
    const int64_t row = (tg / G) * kTileRows + lane;
    packed[w] = row < rows ? canonical[(row * G + g) * kBlockWords + j] : 0u;
}

// ---------------------------------------------------------------------------
// The reference's tiled pair <-> packed words (an exact byte permutation,
// src/ternel_mlx/packing.py:51-83 composed with the packed-word interleave):
// codes[r / tile][g][s][r % tile] is block byte 2 + s of block (r, g),
// scales[r / tile][g][r % tile] its bytes 0-1. One thread per packed word.
// The upload also counts illegal code bytes exactly as validate_packed_codes
// (src/ternel_mlx/packing.py:29-48) does: slots 0..24 above 242, slot 25
// above 26.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(kThreads) void words_from_tiled_kernel(const uint8_t *__restrict__ codes,
                                                                    const uint16_t *__restrict__ scales,
                                                                    uint32_t *__restrict__ packed, int64_t rows,
                                                                    int64_t G, int64_t tile, int64_t total_words,
                                                                    unsigned long long *counters) {
    const int64_t w = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    uint32_t bad_regular = 0, bad_tail = 0;
    if (w < total_words) {
        const int lane = static_cast<int>(w % kTileRows);
        const int64_t rest = w / kTileRows;
        const int j = static_cast<int>(rest % kBlockWords);
        const int64_t tg = rest / kBlockWords;
        const int64_t g = tg % G;
        const int64_t row = (tg / G) * kTileRows + lane;
        uint32_t word = 0;
        if (row < rows) {
            const int64_t tt = row / tile, rr = row % tile;
            const uint8_t *code = codes + ((tt * G + g) * kCodeSlots) * tile + rr;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int byte = 4 * j + i;
                uint32_t v;
                if (byte < 2) {
                    v = (scales[(tt * G + g) * tile + rr] >> (8 * byte)) & 0xffu;
                } else {
                    const int slot = byte - 2;
                    v = code[slot * tile];
                    if (slot < kFullSlots) bad_regular += v > 242u;
                    else bad_tail += v > kMaxTailByte;
                }
                word |= v << (8 * i);
            }
        }
        packed[w] = word;
    }
    bad_regular = wave_sum_u32(bad_regular);
    bad_tail = wave_sum_u32(bad_tail);
    if ((threadIdx.x & 63) == 0) {
        if (bad_regular) atomicAdd(&counters[0], static_cast<unsigned long long>(bad_regular));
        if (bad_tail) atomicAdd(&counters[1], static_cast<unsigned long long>(bad_tail));
    }
}

__global__ __launch_bounds__(kThreads) void tiled_from_words_kernel(const uint32_t *__restrict__ packed,
                                                                    uint8_t *__restrict__ codes,
                                                                    uint16_t *__restrict__ scales, int64_t rows,
                                                                    int64_t G, int64_t tile, int64_t total_words) {
    const int64_t w = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (w >= total_words) return;
    const int lane = static_cast<int>(w % kTileRows);
    const int64_t rest = w / kTileRows;
    const int j = static_cast<int>(rest % kBlockWords);
    const int64_t tg = rest / kBlockWords;
    const int64_t g = tg % G;
    const int64_t row = (tg / G) * kTileRows + lane;
    if (row >= rows) return;
    const uint32_t word = packed[w];
    const int64_t tt = row / tile, rr = row % tile;
    if (j == 0) scales[(tt * G + g) * tile + rr] = static_cast<uint16_t>(word & 0xffffu);
    uint8_t *code = codes + ((tt * G + g) * kCodeSlots) * tile + rr;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int byte = 4 * j + i;
        if (byte >= 2) code[(byte - 2) * tile] = static_cast<uint8_t>(word >> (8 * i));
    }
}

__global__ __launch_bounds__(kThreads) void deinterleave_kernel(const uint32_t *__restrict__ packed,
                                                                uint32_t *__restrict__ canonical, int64_t G,
                                                                int64_t total_words) {
    const int64_t c = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (c >= total_words) return;
    const int j = static_cast<int>(c % kBlockWords);
    const int64_t rg = c / kBlockWords;
    const int64_t g = rg % G;
    const int64_t row = rg / G;
    canonical[c] = packed[packed_word_index(row, G, g, j)];
}

// ---------------------------------------------------------------------------
// get_rows_kernel: one thread per (token, group, run of 8 weights) writes its
// run with one 16-byte store (two for fp32): each value (t - 1) * scale,
// evaluated in fp32 and rounded to T (exact for fp16 and fp32). Weight w of a
// block is digit w % 5 of code byte w / 5 -- the tail byte is code byte 25,
// its digits 0-2 weights 125-127 -- so a run reads the scale word and the two
// words that hold its two or three code bytes, and takes its digits from a
// table of each byte's five base-3 digits (2 bits each) in LDS. Ids outside
// [0, rows) give zeros (src/ternel_mlx/kernels.py:869-880). CANON: the table
// is canonical block rows (row r, group g at byte (r * G + g) * 28), so a
// token's 1,120 bytes are one contiguous run; else the packed layout, where a
// row's words lie in separate 256-byte segments.
// ---------------------------------------------------------------------------
constexpr int kGatherRuns = kBlockWeights / 8;  // 8-weight runs per block
typedef uint32_t gather_u32x4 __attribute__((vector_size(16)));

template <typename T, bool CANON>
__global__ __launch_bounds__(kThreads) void get_rows_kernel(const uint32_t *__restrict__ packed,
                                                            int64_t rows, int G,
                                                            const int64_t *__restrict__ ids,
                                                            int64_t n_ids, T *__restrict__ out,
                                                            int vector_out) {
    __shared__ uint32_t digits[256];  // byte b -> its digits, digit i in bits 2i..2i+1
    digits[threadIdx.x] = tq1_bytes::byte_digits(threadIdx.x);
    __syncthreads();
    const int64_t per_token = static_cast<int64_t>(G) * kGatherRuns;
    const int64_t total = n_ids * per_token;
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x; i < total;
         i += static_cast<int64_t>(gridDim.x) * kThreads) {
        const int64_t t = i / per_token;
        const int rem = static_cast<int>(i - t * per_token);
        const int g = rem / kGatherRuns;
        const int k = rem - g * kGatherRuns;
        const int64_t id = ids[t];
        float v[8];
        if (id < 0 || id >= rows) {
#pragma unroll
            for (int e = 0; e < 8; ++e) v[e] = 0.0f;
        } else {
            const int w0 = 8 * k;
            const int b0 = w0 / 5;       // first code byte of the run
            const int phase = w0 - 5 * b0;  // its first digit
            const int byte0 = 2 + b0;    // byte offset in the 28-byte block
            const int word = byte0 >> 2;
            auto word_at = [&](int j) {
                return CANON ? packed[(id * G + g) * kBlockWords + j] : packed[packed_word_index(id, G, g, j)];
            };
            const float scale = half_bits_to_float(word_at(0));
            const uint32_t lo = word_at(word);
            // A run never needs a byte past the block: k = 14, 15 use two bytes.
            const uint32_t hi = word + 1 < kBlockWords ? word_at(word + 1) : 0u;
            const uint64_t window = ((static_cast<uint64_t>(hi) << 32) | lo) >> ((byte0 & 3) * 8);
            const uint32_t d = digits[window & 0xffu] | (digits[(window >> 8) & 0xffu] << 10) |
                               (digits[(window >> 16) & 0xffu] << 20);
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const uint32_t trit = (d >> (2 * (phase + e))) & 3u;
                v[e] = (static_cast<float>(trit) - 1.0f) * scale;
            }
        }
        T *o = out + t * static_cast<int64_t>(G) * kBlockWeights + g * kBlockWeights + 8 * k;
        if (vector_out) {
            if constexpr (sizeof(T) == 4) {
                reinterpret_cast<float4 *>(o)[0] = float4{v[0], v[1], v[2], v[3]};
                reinterpret_cast<float4 *>(o)[1] = float4{v[4], v[5], v[6], v[7]};
            } else {
                uint32_t pk[4];
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    pk[e] = static_cast<uint32_t>(__builtin_bit_cast(uint16_t, from_f32<T>(v[2 * e]))) |
                            (static_cast<uint32_t>(__builtin_bit_cast(uint16_t, from_f32<T>(v[2 * e + 1]))) << 16);
                // Non-temporal: a wave's store is one contiguous 1 KiB that no
                // cache needs (8192-token fp16 gather 25.4 -> 21.7 us on MI355X;
                // the fp32 form's two 16-byte stores per lane, 32 bytes apart,
                // measured 45 -> 70 us that way, so they keep plain stores).
                __builtin_nontemporal_store(gather_u32x4{pk[0], pk[1], pk[2], pk[3]},
                                            reinterpret_cast<gather_u32x4 *>(o));
            }
        } else {
#pragma unroll
            for (int e = 0; e < 8; ++e) o[e] = from_f32<T>(v[e]);
        }
    }
}

// ---------------------------------------------------------------------------
// lut_gemv_kernel: the LUT23 product (algorithm of src/ternel_mlx/kernels.py
// :244-342), re-designed for wave64 on the packed layout.
//
// Grid (row blocks of 256 = four 64-row tiles, batch tiles of BT, K chunks of
// C groups). Each lane owns one row. The kernel
//   1. issues its row's word loads (one coalesced 256-byte load per wave per
//      word) two blocks ahead of the block it sums, so weights stream while
//   2. the workgroup builds the LUT23 tables of its C groups x BT vectors in
//      LDS: 51 tasks per (vector, group) -- 25 L2 slots, 25 L3 slots, the
//      tail -- each computing its 9 or 27 entries from 2-3 activations;
//   3. per code byte p adds L2[s][p % 9] + L3[s][p / 9] (hi = (p*57) >> 9).
//      All lanes of a wave index the same slot's 9- or 27-entry table, which
//      sit in distinct LDS banks, so every lookup is conflict-free; the table
//      base is a compile-time offset, so a lookup's address is just 4*lo or
//      4*hi. Per group: acc = fma(scale, sum, acc) with the raw fp16 scale --
//      the reference's summation order, so an unsplit launch is bit-exact
//      with it;
//   4. with one K chunk writes y; otherwise writes its fp32 partial, and the
//      last workgroup of the row block to arrive (agent-scope counter) adds
//      the chunks in chunk order -- deterministic -- writes y and re-arms the
//      counter to zero.
// Illegal regular bytes index inside the group's 927 entries and the tail is
// clamped, so no input reads outside the tables.
// ---------------------------------------------------------------------------
// Blocks whose words are in flight ahead of the one being consumed, for a
// wave stream of cb blocks per sub-chunk: one where the stream has two (the
// second issued while the first is summed rather than before the tables:
// gate/up M=1 9.64-9.74 -> 9.24-9.33 us on MI355X, O and out_proj the same),
// two where it has more (down 10.16-10.23 against 10.24-10.32 with one).
constexpr int lut_load_ahead(int cb) { return cb > 2 ? 2 : 1; }

// The sub-chunk's activations (BT vectors x C groups), copied to LDS with
// 16-byte loads (element loads for rows that are not 16-byte aligned): a
// workgroup asks for each of their cache lines once, where per-task gathers
// ask for every line several times (gate/up M=1 9.39 -> 9.28 us on MI355X).
// issue() loads them into registers -- every thread issues its loads, extra
// threads repeating the last piece, so no load sits behind a branch -- and
// store() writes them to LDS once they have arrived.
template <typename T, int C, int BT, int NT>
struct ActivationCopy {
    static constexpr int kRow = C * kBlockWeights;
    static constexpr int kVec = 16 / static_cast<int>(sizeof(T));
    static constexpr int kPieces = BT * kRow / kVec;
    static constexpr int kIters = (kPieces + NT - 1) / NT;
    static constexpr int kElemIters = (BT * kRow + NT - 1) / NT;
    uint4 v[kIters];
    T e[kElemIters];
    bool aligned;

    __device__ __forceinline__ void issue(const T *__restrict__ x, int64_t K, int M, int b0, int g0, int tid) {
        aligned = (reinterpret_cast<uintptr_t>(x) & 15u) == 0;
        if (aligned) {
#pragma unroll
            for (int it = 0; it < kIters; ++it) {
                const int i = min(tid + it * NT, kPieces - 1);
                const int j = i / (kRow / kVec);
                const int q = i - j * (kRow / kVec);
                const T *src = x + static_cast<int64_t>(min(b0 + j, M - 1)) * K +
                               static_cast<int64_t>(g0) * kBlockWeights + q * kVec;
                v[it] = *reinterpret_cast<const uint4 *>(src);
            }
        } else {
#pragma unroll
            for (int it = 0; it < kElemIters; ++it) {
                const int i = min(tid + it * NT, BT * kRow - 1);
                const int j = i / kRow;
                e[it] = x[static_cast<int64_t>(min(b0 + j, M - 1)) * K + static_cast<int64_t>(g0) * kBlockWeights +
                          (i - j * kRow)];
            }
        }
    }
    __device__ __forceinline__ void store(T (*xs)[kRow], int tid) const {
        if (aligned) {
#pragma unroll
            for (int it = 0; it < kIters; ++it) {
                const int i = min(tid + it * NT, kPieces - 1);
                const int j = i / (kRow / kVec);
                *reinterpret_cast<uint4 *>(&xs[j][(i - j * (kRow / kVec)) * kVec]) = v[it];
            }
        } else {
#pragma unroll
            for (int it = 0; it < kElemIters; ++it) {
                const int i = min(tid + it * NT, BT * kRow - 1);
                const int j = i / kRow;
                xs[j][i - j * kRow] = e[it];
            }
        }
    }
};

// The LUT23 tables of one sub-chunk from its staged activations. Per
// (vector, group): 25 L2 tasks (slot s: 9 entries from x[5s], x[5s+1]), and
// 26 three-trit tasks (L3 slot s: 27 entries from x[5s+2..5s+4]; the tail:
// 27 from x[125..127]). The three-trit tasks take threads [0, T3) and the L2
// tasks start at the next multiple of 64, so every wave runs one kind of
// task. A three-trit table is built from its 9 two-trit sums,
// entry e = pair[e % 9] + d[e / 9] -- the reference's (a + b) + d, rounded
// the same way. Entries are (t - 1) * x as real products, so 0 * inf = NaN
// propagates as in the reference.
// The tables lie in two regions: the BT C three-trit table sets (26 tables
// of 27 floats each, 702 floats per (vector, group)) from float 0, then the
// BT C two-trit sets (25 of 9 floats, 225). Task k of a kind writes at k
// times its table size, so a wave's consecutive tasks start in distinct banks.
template <typename T, int C, int BT, int NT>
__device__ __forceinline__ void build_lut_tables(float *lut, const T (*xs)[C * kBlockWeights], int tid) {
    constexpr int kTrit3 = BT * C * (kFullSlots + 1);
    constexpr int kL2Start = (kTrit3 + 63) / 64 * 64;
    constexpr int kTasks = kL2Start + BT * C * kFullSlots;
#pragma unroll
    for (int it = 0; it < (kTasks + NT - 1) / NT; ++it) {
        const int i = tid + it * NT;
        if (i < kTrit3) {
            const int j = i / (C * (kFullSlots + 1));
            const int rem = i - j * (C * (kFullSlots + 1));
            const int c = rem / (kFullSlots + 1);
            const int s = rem - c * (kFullSlots + 1);
            const T *xg = xs[j] + c * kBlockWeights + (s < kFullSlots ? 5 * s + 2 : 125);
            const float x0 = to_f32<T>(xg[0]), x1 = to_f32<T>(xg[1]), x2 = to_f32<T>(xg[2]);
            const float a[3] = {-1.0f * x0, 0.0f * x0, 1.0f * x0};
            const float b[3] = {-1.0f * x1, 0.0f * x1, 1.0f * x1};
            const float d[3] = {-1.0f * x2, 0.0f * x2, 1.0f * x2};
            float pair[kL2Entries];
#pragma unroll
            for (int e = 0; e < kL2Entries; ++e) pair[e] = a[e % 3] + b[e / 3];
            float *dst = lut + i * kL3Entries;  // (j C + c) 702 + 27 s, the tail as slot 25
#pragma unroll
            for (int e = 0; e < kL3Entries; ++e) dst[e] = pair[e % 9] + d[e / 9];
        } else if (i >= kL2Start && i < kTasks) {
            const int t = i - kL2Start;
            const int j = t / (C * kFullSlots);
            const int rem = t - j * (C * kFullSlots);
            const int c = rem / kFullSlots;
            const int s = rem - c * kFullSlots;
            const T *xg = xs[j] + c * kBlockWeights + 5 * s;
            const float x0 = to_f32<T>(xg[0]), x1 = to_f32<T>(xg[1]);
            const float a[3] = {-1.0f * x0, 0.0f * x0, 1.0f * x0};
            const float b[3] = {-1.0f * x1, 0.0f * x1, 1.0f * x1};
            float *dst = lut + BT * C * kLut3Floats + t * kL2Entries;  // then (j C + c) 225 + 9 s
#pragma unroll
            for (int e = 0; e < kL2Entries; ++e) dst[e] = a[e % 3] + b[e / 3];
        }
    }
}

// LUT23 split of the 25 code bytes of a block, two bytes per 16-bit-packed
// operation: hi = (p * 57) >> 9 == p / 9 (exact for p <= 511), lo = p - 9 hi.
// Each 16-bit digit becomes a table byte address with one multiply-add that
// selects its half (v_mad_u32_u16 with op_sel): 4 * digit + base, where base is
// the wave's table base; slot and block offsets go in the reads' immediates.
typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));

__device__ __forceinline__ uint32_t lut_address_lo(uint32_t pair, uint32_t base) {
    uint32_t r;
    asm("v_mad_u32_u16 %0, %1, 4, %2" : "=v"(r) : "v"(pair), "v"(base));
    return r;
}
__device__ __forceinline__ uint32_t lut_address_hi(uint32_t pair, uint32_t base) {
    uint32_t r;
    asm("v_mad_u32_u16 %0, %1, 4, %2 op_sel:[1,0,0,0]" : "=v"(r) : "v"(pair), "v"(base));
    return r;
}

// a * b + c and a * b for a, b below 2^24 (v_mad_u32_u24 / v_mul_u32_u24).
// Written out because the compiler turns a 32-bit multiply-add into a 64-bit
// v_mad_u64_u32 whose unused high addend the register allocator may place in
// a register with a load still in flight, and then waits for that load.
__device__ __forceinline__ uint32_t mad_u24(uint32_t a, uint32_t b, uint32_t c) {
    uint32_t r;
    asm("v_mad_u32_u24 %0, %1, %2, %3" : "=v"(r) : "v"(a), "v"(b), "v"(c));
    return r;
}
__device__ __forceinline__ uint32_t mul_u24(uint32_t a, uint32_t b) {
    uint32_t r;
    asm("v_mul_u32_u24 %0, %1, %2" : "=v"(r) : "v"(a), "v"(b));
    return r;
}

__device__ __forceinline__ void split_pair(uint32_t pair, uint32_t base_lo, uint32_t base_hi, uint32_t &lo_a,
                                           uint32_t &hi_a, uint32_t &lo_b, uint32_t &hi_b) {
    const u16x2 p = __builtin_bit_cast(u16x2, pair);
    const u16x2 h = tq1_bytes::lut23_high(p);
    const u16x2 l = tq1_bytes::lut23_low(p, h);
    const uint32_t hb = __builtin_bit_cast(uint32_t, h), lb = __builtin_bit_cast(uint32_t, l);
    lo_a = lut_address_lo(lb, base_lo);
    hi_a = lut_address_lo(hb, base_hi);
    lo_b = lut_address_hi(lb, base_lo);
    hi_b = lut_address_hi(hb, base_hi);
}

// All four bytes of a block word: table byte addresses lo/hi for byte b of the
// word. Bytes 1 and 3 move to the 16-bit halves with one byte permute
// (selector 0x0c = zero). The two-trit digits index from base_lo, the
// three-trit ones from base_hi.
__device__ __forceinline__ void split_word(uint32_t word, uint32_t base_lo, uint32_t base_hi, uint32_t (&lo)[4],
                                           uint32_t (&hi)[4]) {
    split_pair(word & 0x00ff00ffu, base_lo, base_hi, lo[0], hi[0], lo[2], hi[2]);  // bytes 0 and 2
    split_pair(__builtin_amdgcn_perm(0u, word, 0x0c030c01u), base_lo, base_hi, lo[1], hi[1], lo[3],
               hi[3]);  // bytes 1 and 3
}
__device__ __forceinline__ void split_word(uint32_t word, uint32_t base, uint32_t (&lo)[4], uint32_t (&hi)[4]) {
    split_word(word, base, base, lo, hi);
}

// Adds partial[0..k) (stride apart) left to right. The agent-coherent loads of
// up to 32 chunks are all issued before the first add, so a split costs one
// memory round trip here rather than one per chunk.
__device__ __forceinline__ float sum_partials_in_order(const float *src, int64_t stride, int k) {
    constexpr int kBatch = 32;
    float a = 0.0f;
    for (int z0 = 0; z0 < k; z0 += kBatch) {
        float v[kBatch];
#pragma unroll
        for (int u = 0; u < kBatch; ++u)
            v[u] = z0 + u < k ? __hip_atomic_load(src + (z0 + u) * stride, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)
                              : 0.0f;
        if (z0 == 0) {
            a = v[0];
#pragma unroll
            for (int u = 1; u < kBatch; ++u)
                if (u < k) a += v[u];
        } else {
#pragma unroll
            for (int u = 0; u < kBatch; ++u)
                if (z0 + u < k) a += v[u];
        }
    }
    return a;
}

// s_waitcnt with vmcnt(0) and the other counters left alone (gfx9 encoding).
__device__ __forceinline__ void wait_vector_memory() { __builtin_amdgcn_s_waitcnt(0x0f70); }

// SiLU(g) * u of a gate/up pair, in fp32 from the two outputs as the unfused
// layers would round them (the activation type): the elementwise step of a
// SwiGLU MLP applied to the linear's outputs.
template <typename T>
__device__ __forceinline__ T swiglu_pair(T gate, T up) {
    const float g = to_f32<T>(gate);
    return from_f32<T>(g / (1.0f + expf(-g)) * to_f32<T>(up));
}

// RT 64-row tiles per workgroup (4, or 2 where 256-row blocks would leave
// fewer than about 1.5 workgroups per CU).
template <typename T, int C, int BT, bool GLU = false, int KW = 1, int RT = kThreads / kTileRows>
__global__ __launch_bounds__(RT * kTileRows * KW) void lut_gemv_kernel(
    const uint32_t *__restrict__ packed, const T *__restrict__ x, T *__restrict__ y,
    float *__restrict__ partial, unsigned *__restrict__ counters, int M, int N, int G, int chunk_groups,
    int k_split) {
    // KW waves share each 64-row tile: wave stream s sums blocks
    // [s * CB, (s + 1) * CB) of every sub-chunk, so all of a sub-chunk's words
    // can be in flight from the start without one wave stalling on their issue.
    // Streams above 0 hand their block sums and scales to stream 0 through LDS,
    // which folds them into acc in block order: the summation order (and so the
    // result) does not depend on KW.
    // (Four waves per tile measured slower: a 1024-thread workgroup leaves too
    // few resident per CU.)
    static_assert(KW == 1 || KW == 2, "one or two waves per row tile");
    static_assert(C % KW == 0, "each wave stream takes whole blocks");
    static_assert(RT == 2 || RT == 4, "128- or 256-row workgroups");
    constexpr int RB = RT * kTileRows;  // rows per workgroup (threads per wave stream)
    constexpr int NT = RB * KW;
    constexpr int CB = C / KW;
    constexpr int LA = lut_load_ahead(CB);
    __shared__ float lut[BT][C][kLutFloats];
    __shared__ __align__(16) T xs[BT][C * kBlockWeights];
    __shared__ float2 xchg[KW > 1 ? (KW - 1) * CB * BT : 1][RB];
    __shared__ unsigned s_last;

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int stream = __builtin_amdgcn_readfirstlane(tid / RB);  // wave-uniform, branched on as such
    const int tile = blockIdx.x * RT + ((tid & (RB - 1)) >> 6);
    const int row = tile * kTileRows + lane;
    const bool row_ok = row < N && stream == 0;  // lanes that hold and write the result
    const int b0 = blockIdx.y * BT;
    const int g_begin = blockIdx.z * chunk_groups;
    const int g_end = g_begin + chunk_groups;
    const int64_t K = static_cast<int64_t>(G) * kBlockWeights;
    // Waves past the last tile load (and discard) the last tile instead of
    // branching around their loads.
    const int load_tile = min(tile, (N + kTileRows - 1) / kTileRows - 1);
    const uint32_t *row_words = packed + static_cast<int64_t>(load_tile) * G * kTileGroupWords + lane;
    const int lut_wave_id =
        ((blockIdx.z * gridDim.y + blockIdx.y) * gridDim.x + blockIdx.x) * KW * RT + (tid >> 6);
    (void)lut_wave_id;
    TQ1_PHASE(lut_wave_id, 0);  // wave start
    TQ1_PHASE_XCC(lut_wave_id);

    float acc[BT];
#pragma unroll
    for (int j = 0; j < BT; ++j) acc[j] = 0.0f;

    // The work of one wave stream -- blocks [stream * CB, (stream + 1) * CB) of
    // every sub-chunk. One copy of the code serves every stream, whose word
    // loads and table reads start from its own base: a copy per stream (table
    // offsets as immediates) doubled the code for the same speed. Per sub-chunk
    // of C groups:
    //   1. the activations of this thread's table tasks, then this row's
    //      blocks: only the first LA blocks' words are issued before the
    //      tables, block c + LA as block c is consumed -- a wave
    //      that issued all of its loads at once would stall on issue while the
    //      CU's memory queue drains, and reach its first sum only then;
    //   2. the tables, after every lane is done reading the previous ones;
    //   3. the blocks, in load order (loads complete in order; rows past N
    //      compute a discarded value). Within a block: slot 0..24, the tail,
    //      then one fma with the scale; blocks fold into acc in order -- the
    //      reference's summation order. Streams above 0 leave their block sums
    //      and scales in LDS; stream 0 folds them after a barrier.
    const int cb0 = stream * CB;  // first block of this wave's stream
    const char *const lut_bytes = reinterpret_cast<const char *>(&lut[0][0][0]);
    // This stream's first three-trit and two-trit table sets (build_lut_tables'
    // two regions).
    const uint32_t base3 = static_cast<uint32_t>(cb0 * kLut3Floats * 4);
    const uint32_t base2 = static_cast<uint32_t>((BT * C * kLut3Floats + cb0 * kLut2Floats) * 4);
    auto table3 = [&](uint32_t address, int j, int c, int entry) {
        return *reinterpret_cast<const float *>(lut_bytes + address + ((j * C + c) * kLut3Floats + entry) * 4);
    };
    auto table2 = [&](uint32_t address, int j, int c, int entry) {
        return *reinterpret_cast<const float *>(lut_bytes + address + ((j * C + c) * kLut2Floats + entry) * 4);
    };
    auto run = [&](int g0) {
        const uint32_t *wp = row_words + (static_cast<int64_t>(g0) * kBlockWords + cb0 * kBlockWords) * kTileRows;
        uint32_t w[CB][kBlockWords];
#pragma unroll
        for (int c = 0; c < (LA < CB ? LA : CB); ++c)
#pragma unroll
            for (int j = 0; j < kBlockWords; ++j) w[c][j] = wp[(c * kBlockWords + j) * kTileRows];
        __builtin_amdgcn_sched_barrier(0);
        if (g0 == g_begin) TQ1_PHASE(lut_wave_id, 2);  // first words issued
        // (With several streams the fold barrier below already orders the
        // previous sub-chunk's table and exchange reads before this.)
        if (KW == 1 && g0 != g_begin) __syncthreads();
        build_lut_tables<T, C, BT, NT>(&lut[0][0][0], xs, tid);
        if (g0 == g_begin) TQ1_PHASE(lut_wave_id, 3);  // own table entries written
        __syncthreads();
        if (g0 == g_begin) TQ1_PHASE(lut_wave_id, 4);  // tables ready
#pragma unroll
        for (int c = 0; c < CB; ++c) {
            if (c + LA < CB) {
#pragma unroll
                for (int j = 0; j < kBlockWords; ++j)
                    w[c + LA][j] = wp[((c + LA) * kBlockWords + j) * kTileRows];
            }
            __builtin_amdgcn_sched_barrier(0);
            // The sum starts at slot 0's pair rather than at 0 + pair: equal
            // except that a -0 pair stays -0, which the fma into acc (from +0)
            // turns into the same +0.
            float sum[BT];
#pragma unroll
            for (int word = 0; word < kBlockWords; ++word) {
                uint32_t lo[4], hi[4];
                split_word(w[c][word], base2, base3, lo, hi);
#pragma unroll
                for (int b = 0; b < 4; ++b) {
                    const int s = word * 4 + b - 2;  // code byte s is block byte 2 + s
                    if (s < 0 || s >= kFullSlots) continue;
#pragma unroll
                    for (int j = 0; j < BT; ++j) {
                        const float pair =
                            table2(lo[b], j, c, s * kL2Entries) + table3(hi[b], j, c, s * kL3Entries);
                        sum[j] = s == 0 ? pair : sum[j] + pair;
                    }
                }
            }
            const float scale = half_bits_to_float(w[c][0]);
            const uint32_t tail = base3 + 4 * tq1_bytes::tail_entry(w[c][6] >> 24);
#pragma unroll
            for (int j = 0; j < BT; ++j) {
                sum[j] += table3(tail, j, c, kFullSlots * kL3Entries);
                if (KW == 1 || stream == 0)
                    acc[j] = fmaf(scale, sum[j], acc[j]);
                else
                    xchg[((stream - 1) * CB + c) * BT + j][tid & (RB - 1)] = make_float2(sum[j], scale);
            }
            __builtin_amdgcn_sched_barrier(0);
        }
        if constexpr (KW > 1) {
            __syncthreads();
            if (stream == 0) {
#pragma unroll
                for (int c = 0; c < (KW - 1) * CB; ++c)
#pragma unroll
                    for (int j = 0; j < BT; ++j) {
                        const float2 v = xchg[c * BT + j][tid];
                        acc[j] = fmaf(v.y, v.x, acc[j]);
                    }
            }
        }
    };
    for (int g0 = g_begin; g0 < g_end; g0 += C) {
        // Activations first, copied to LDS and waited for before any word is
        // issued. Their lines are first read from HBM, where the chip-wide
        // burst of word loads would queue ahead of them: issued just ahead
        // of the words (no wait), the first waves of an XCC had them at
        // 0.9 us instead of 0.5 (gate/up 9.28 -> 9.87 us on MI355X); read
        // with scalar loads, 2.1 us.
        ActivationCopy<T, C, BT, NT> copy;
        copy.issue(x, K, M, b0, g0, tid);
        copy.store(xs, tid);
        if (g0 == g_begin) TQ1_PHASE(lut_wave_id, 1);  // own activation copies arrived
        __syncthreads();
        run(g0);
    }

    TQ1_PHASE(lut_wave_id, 5);  // all blocks summed
    // 4. Output. With GLU, rows 2r and 2r+1 are the gate and up rows of one
    // SwiGLU unit and sit in adjacent lanes: each lane rounds its value as the
    // unfused linear would, the even lane takes its partner's and writes
    // SiLU(gate) * up to y[r] of an N/2-wide output. Every lane takes part in
    // the exchange.
    auto store = [&](int j, float v) {
        if constexpr (GLU) {
            const T own = from_f32<T>(v);
            const float partner = __shfl_xor(to_f32<T>(own), 1, 64);
            if (row_ok && (lane & 1) == 0 && b0 + j < M)
                y[static_cast<int64_t>(b0 + j) * (N / 2) + row / 2] = swiglu_pair<T>(own, from_f32<T>(partner));
        } else {
            if (row_ok && b0 + j < M) y[static_cast<int64_t>(b0 + j) * N + row] = from_f32<T>(v);
        }
    };
    if (k_split == 1) {
#pragma unroll
        for (int j = 0; j < BT; ++j) store(j, acc[j]);
        return;
    }
    // Split: publish the partial with agent-scope atomic stores (sc1: written
    // through to the device's coherence point, past the per-XCD L2), wait until
    // every one is acknowledged there (vmcnt(0)), then count this chunk in with
    // a relaxed agent-scope atomic. The workgroup that brings the count to
    // k_split reads the chunks with agent-scope atomic loads (sc1: from the
    // coherence point) and adds them in chunk order. This is the instruction
    // sequence of an agent-scope release/acquire hand-off on gfx950 without
    // the L2 writeback and invalidate, which concern only data written without
    // sc1 -- and this hand-off writes none. The compiler barriers keep the
    // count from moving above the wait. (A {value, flag} slot protocol that
    // needs no acknowledgement measured 9.6 -> 10.9 us for gate/up on
    // MI355X; a __threadfence version about 60 us.)
    if (row_ok) {
#pragma unroll
        for (int j = 0; j < BT; ++j)
            if (b0 + j < M)
                __hip_atomic_store(partial + (static_cast<int64_t>(blockIdx.z) * M + b0 + j) * N + row, acc[j],
                                   __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    asm volatile("" ::: "memory");
    wait_vector_memory();
    asm volatile("" ::: "memory");
    TQ1_PHASE(lut_wave_id, 6);  // partial stored and acknowledged
    __syncthreads();
    unsigned *counter = counters + static_cast<int64_t>(blockIdx.y) * gridDim.x + blockIdx.x;
    if (tid == 0)
        s_last = __hip_atomic_fetch_add(counter, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
                 static_cast<unsigned>(k_split - 1);
    __syncthreads();
    TQ1_PHASE(lut_wave_id, 7);  // arrival counted
    if (!s_last) return;
    const int64_t stride = static_cast<int64_t>(M) * N;
#pragma unroll
    for (int j = 0; j < BT; ++j) {
        const float *src = partial + static_cast<int64_t>(b0 + j) * N + row;
        store(j, row_ok && b0 + j < M ? sum_partials_in_order(src, stride, k_split) : 0.0f);
    }
    if (tid == 0) __hip_atomic_store(counter, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    TQ1_PHASE(lut_wave_id, 8);  // fix-up done
}

// ---------------------------------------------------------------------------
// strip_gemv_kernel: the M = 1 decode GEMV (one activation vector) for
// matrices of at most kStripMaxGroups groups per row (K <= 5120) and at most
// 96 rows per CU, with every row's K reduction inside one workgroup (the
// LUT23 algorithm of src/ternel_mlx/kernels.py:244-342). With SPLIT, rows of
// more than 40 groups: Z <= 4 workgroups per strip each take one K chunk of
// at most 40 groups, and each row's Z partials meet in exchange slots (the
// epilogue below).
//
// One workgroup per CU owns a strip of R <= 96 rows: strip s of S holds rows
// [2 floor(s U / S), 2 floor((s + 1) U / S)), U = ceil(N / 2), so strips
// differ by at most two rows and a gate/up pair never straddles two of them.
// Workgroup b takes strip (b % 8) P / 8 + b / 8 when P is a multiple of 8:
// workgroups are dealt to the eight XCDs in turn, so each XCD holds adjacent
// strips and a cache line shared by two strips is read into one L2.
// The workgroup stages the activations in LDS (one 16-byte load per thread;
// no wave requests a weight word until every wave's activations are in LDS,
// as a wave's activation load queued behind its CU's word loads comes back
// microseconds later) and builds the LUT23
// tables of all G groups once (G x 927 floats, 148,320 bytes at G = 40);
// they stay for the whole launch, so a lane may look up any group. The
// strip's R x G blocks are numbered t = g R + i (row i, group g), so
// consecutive lanes read consecutive rows of one group, and cut into items
// of 64; wave w takes items w, w + 16, ... (so each SIMD's four waves hold
// equal shares), with its first item's words requested before the tables are
// built and the next item's as it sums one. Every load is issued
// unconditionally (past the end of a run a wave re-reads the item it sums,
// from cache), so the compiler's wait counts stay exact: a wait for one item
// never waits for the next.
// Sums: a block's in the reference's slot order; its scale * sum stored
// alone; a row's G values in eight contiguous group ranges, each in group
// order by one of eight adjacent lanes, and the eight partials added across
// the lanes with DPP. The order is fixed by the shape, so results are bit-identical from
// run to run, and equal the reference's to within fp32 reassociation of the
// per-group terms.
// No workspace, no memory shared between workgroups.
// (Above 96 rows per CU the (tile, group) LUT23 kernel above runs: its 2-3
// workgroups per CU overlap one workgroup's table build with another's sums,
// which at more than 96 rows outweighs the split-K hand-off this avoids.)
// ---------------------------------------------------------------------------
constexpr int kStripWaves = 16;
constexpr int kStripThreads = kStripWaves * 64;
constexpr int kStripMaxGroups = 40;
constexpr int kStripMaxRows = 96;
constexpr int kStripLdsFloats = 40960;  // 160 KiB, the workgroup limit
// The tables of all groups in two regions: every group's 26 three-trit
// tables (27 floats each, the tail last) from float 0, then every group's 25
// two-trit tables (9 floats each). Task k of a kind writes at k times its
// table size, so a wave's 64 consecutive tasks start in 64 different banks
// (27 and 9 are odd).
constexpr int kStripL3Floats = kLut3Floats;  // 702 per group
constexpr int kStripL2Floats = kLut2Floats;  // 225 per group
static_assert(kStripMaxGroups * kLutFloats + kStripMaxGroups * kStripMaxRows <= kStripLdsFloats, "LDS fits");
constexpr int kStripTrit3Iters = (kStripMaxGroups * (kFullSlots + 1) + kStripThreads - 1) / kStripThreads;
constexpr int kStripL2Iters = (kStripMaxGroups * kFullSlots + kStripThreads - 1) / kStripThreads;
// Below this many rows the LUT23 kernel is used instead (equal speed).
constexpr int kStripMinRows = 2048;

struct StripGeometry {
    int N, G;        // rows, groups per row
    int P;           // workgroups: S strips x Z K chunks
    int S, Z;        // strips; K chunks of at most Gc groups (Z = 1: no split)
    int Gc;
    int units;       // U = ceil(N / 2)
    int value_base;  // LDS float offset of the block values (and, before them, the staged activations)
};

// First row of strip s.
__device__ __forceinline__ int strip_row(int s, const StripGeometry &geo) {
    return min(geo.N, 2 * static_cast<int>(static_cast<unsigned>(s * geo.units) / static_cast<unsigned>(geo.S)));
}

// The table tasks of one thread: three-trit task t < 26 G is (group t / 26,
// slot t % 26; slot 25 the tail), two-trit task t < 25 G is (group t / 25,
// slot t % 25). gather() reads their activations (from LDS or global memory,
// every read issued, indices clamped), build() writes the tables from them,
// as build_lut_tables computes them, task t of a kind at t times its table
// size in that kind's region.
template <typename T>
struct StripTasks {
    T v3[kStripTrit3Iters][3], v2[kStripL2Iters][2];

    __device__ __forceinline__ void gather(const T *xs, int G, int tid) {
#pragma unroll
        for (int it = 0; it < kStripTrit3Iters; ++it) {
            const int t = min(tid + it * kStripThreads, G * (kFullSlots + 1) - 1);
            const int g = t / (kFullSlots + 1), s = t - g * (kFullSlots + 1);
            const T *p = xs + g * kBlockWeights + (s < kFullSlots ? 5 * s + 2 : 125);
            v3[it][0] = p[0];
            v3[it][1] = p[1];
            v3[it][2] = p[2];
        }
#pragma unroll
        for (int it = 0; it < kStripL2Iters; ++it) {
            const int t = min(tid + it * kStripThreads, G * kFullSlots - 1);
            const int g = t / kFullSlots, s = t - g * kFullSlots;
            const T *p = xs + g * kBlockWeights + 5 * s;
            v2[it][0] = p[0];
            v2[it][1] = p[1];
        }
    }

    __device__ __forceinline__ void build(float *lut, int G, int tid) const {
#pragma unroll
        for (int it = 0; it < kStripTrit3Iters; ++it) {
            const int t = tid + it * kStripThreads;
            if (t < G * (kFullSlots + 1)) {
                const float x0 = to_f32<T>(v3[it][0]), x1 = to_f32<T>(v3[it][1]), x2 = to_f32<T>(v3[it][2]);
                const float a[3] = {-1.0f * x0, 0.0f * x0, 1.0f * x0};
                const float b[3] = {-1.0f * x1, 0.0f * x1, 1.0f * x1};
                const float d[3] = {-1.0f * x2, 0.0f * x2, 1.0f * x2};
                float pair[kL2Entries];
#pragma unroll
                for (int e = 0; e < kL2Entries; ++e) pair[e] = a[e % 3] + b[e / 3];
                float *dst = lut + t * kL3Entries;  // the three-trit region's g * 702 + 27 s
#pragma unroll
                for (int e = 0; e < kL3Entries; ++e) dst[e] = pair[e % 9] + d[e / 9];
            }
        }
#pragma unroll
        for (int it = 0; it < kStripL2Iters; ++it) {
            const int t = tid + it * kStripThreads;
            if (t < G * kFullSlots) {
                const float x0 = to_f32<T>(v2[it][0]), x1 = to_f32<T>(v2[it][1]);
                const float a[3] = {-1.0f * x0, 0.0f * x0, 1.0f * x0};
                const float b[3] = {-1.0f * x1, 0.0f * x1, 1.0f * x1};
                float *dst = lut + G * kStripL3Floats + t * kL2Entries;  // the two-trit region's g * 225 + 9 s
#pragma unroll
                for (int e = 0; e < kL2Entries; ++e) dst[e] = a[e % 3] + b[e / 3];
            }
        }
    }
};

// One block's LUT23 sum from its words and its group's two-trit and
// three-trit tables at byte offsets `table2` and `table3`: slot 0..24 in
// order, then the tail (the reference's order).
__device__ __forceinline__ float strip_block_sum(const uint32_t (&w)[kBlockWords], const char *lds, uint32_t table2,
                                                 uint32_t table3) {
    auto at = [&](uint32_t address, int entry) {
        return *reinterpret_cast<const float *>(lds + address + entry * 4);
    };
    float sum = 0.0f;
#pragma unroll
    for (int word = 0; word < kBlockWords; ++word) {
        uint32_t lo[4], hi[4];
        split_word(w[word], table2, table3, lo, hi);
#pragma unroll
        for (int b = 0; b < 4; ++b) {
            const int s = word * 4 + b - 2;  // code byte s is block byte 2 + s
            if (s < 0 || s >= kFullSlots) continue;
            const float pair = at(lo[b], s * kL2Entries) + at(hi[b], s * kL3Entries);
            sum = s == 0 ? pair : sum + pair;
        }
    }
    return sum + at(table3 + 4 * tq1_bytes::tail_entry(w[6] >> 24), kFullSlots * kL3Entries);
}

// STAGE: the activations are a 2-byte type at a 16-byte aligned address and
// are staged in LDS with one 16-byte load per thread; otherwise each thread
// reads its table tasks' activations from global memory.
template <typename T, bool GLU, bool STAGE, int PAIRS, bool SPLIT>
__global__ __launch_bounds__(kStripThreads, 1) void strip_gemv_kernel(const uint32_t *__restrict__ packed,
                                                                      const T *__restrict__ x, T *__restrict__ y,
                                                                      unsigned *__restrict__ slots,
                                                                      StripGeometry geo) {
    static_assert(!(SPLIT && GLU), "the fused SwiGLU form is not split");
    __shared__ __align__(16) float lds_f[kStripLdsFloats];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int b = blockIdx.x;
    const int strip_wave_id = b * kStripWaves + wave;
    (void)strip_wave_id;
    TQ1_PHASE(strip_wave_id, 0);
    TQ1_PHASE_XCC(strip_wave_id);

    // Workgroup order: b takes (b % 8) P / 8 + b / 8 where P is a multiple of
    // 8, so each XCD holds a contiguous run; that index is strip u / Z, K
    // chunk u % Z (a strip's chunks run on one XCD).
    const int u = (geo.P & 7) == 0 ? (b & 7) * (geo.P >> 3) + (b >> 3) : b;
    const int s = SPLIT ? u / geo.Z : u;
    const int z = SPLIT ? u - s * geo.Z : 0;
    const int g_lo = z * geo.Gc;                           // first group of this chunk
    const int G = SPLIT ? min(geo.Gc, geo.G - g_lo) : geo.G;  // this workgroup's groups
    x += static_cast<int64_t>(g_lo) * kBlockWeights;

    // Activations first.
    constexpr int kVec = 16 / static_cast<int>(sizeof(T));
    static_assert(!STAGE || sizeof(T) == 2, "staging takes 2-byte activations");
    const int pieces = G * (kBlockWeights / kVec);
    StripTasks<T> tasks;
    uint4 piece;
    if constexpr (STAGE)
        piece = reinterpret_cast<const uint4 *>(x)[min(tid, pieces - 1)];
    else
        tasks.gather(x, G, tid);

    const int lo = strip_row(s, geo);
    const int R = strip_row(s + 1, geo) - lo;
    const int RG = R * G;
    const int n_items = (RG + 63) >> 6;
    // Wave w sums items w, w + 16, w + 32, ...: the waves' shares differ by
    // at most one item. Past its last item a wave's loads re-read the last
    // item it owns (a wave that owns none, the strip's last item).
    const int n_own = n_items > wave ? (n_items - wave + kStripWaves - 1) / kStripWaves : 0;
    const int own_last = n_own > 0 ? wave + (n_own - 1) * kStripWaves : n_items - 1;
    auto item_of = [&](int j) __attribute__((always_inline)) { return min(wave + j * kStripWaves, own_last); };
    const float inv_r = 1.0f / static_cast<float>(max(R, 1));

    // Block t = g R + i of item i for this lane (clamped into the strip):
    // its group and its word offset.
    auto block = [&](int item, int &t, int &g) __attribute__((always_inline)) {
        t = (item << 6) + lane;
        const int tc = min(t, max(RG - 1, 0));
        g = static_cast<int>((static_cast<float>(tc) + 0.5f) * inv_r);
        // (Every factor and result here is below 2^24.)
        const uint32_t row = static_cast<uint32_t>(lo + tc) - mul_u24(static_cast<uint32_t>(g), static_cast<uint32_t>(R));
        return static_cast<int>(
            mad_u24(mad_u24(row >> 6, static_cast<uint32_t>(geo.G), static_cast<uint32_t>(g_lo + g)),
                    static_cast<uint32_t>(kTileGroupWords), row & 63u));
    };
    // (The scheduling barriers keep the sums of the item before from moving
    // above the loads, where they would wait for that item's words first.)
    // An item in flight: this lane's block words, its block index t and its
    // group's table byte offset (computed once, at the load).
    struct Item {
        uint32_t w[kBlockWords];
        int t;
        uint32_t table2, table3;
    };
    auto load = [&](int item, Item &it) __attribute__((always_inline)) {
        int g;
        const uint32_t *p = packed + block(item, it.t, g);
        it.table3 = mul_u24(static_cast<uint32_t>(g), kStripL3Floats * 4);
        it.table2 = mad_u24(static_cast<uint32_t>(g), kStripL2Floats * 4, static_cast<uint32_t>(G * kStripL3Floats * 4));
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int j = 0; j < kBlockWords; ++j) it.w[j] = p[j * kTileRows];
        __builtin_amdgcn_sched_barrier(0);
    };

    // The first item's words are in flight while the tables are built (a
    // second item's too measured slower: with every CU's waves issuing, the
    // issue itself waits for the memory queue, and the tables wait behind it).
    // With staged activations they are requested after the staging barrier,
    // so no wave's activation load waits behind its CU's first words.
    wait_vector_memory();
    Item wa, wb;
    if constexpr (STAGE) {
        T *const xs = reinterpret_cast<T *>(lds_f + geo.value_base);
        if (tid < pieces) reinterpret_cast<uint4 *>(xs)[tid] = piece;
        __syncthreads();
        load(item_of(0), wa);
        TQ1_PHASE(strip_wave_id, 1);  // activations arrived, first words issued
        tasks.gather(xs, G, tid);
    } else {
        load(item_of(0), wa);
        TQ1_PHASE(strip_wave_id, 1);  // activations arrived, first words issued
    }
    tasks.build(lds_f, G, tid);
    __syncthreads();
    TQ1_PHASE(strip_wave_id, 2);  // tables ready

    const char *const lds = reinterpret_cast<const char *>(lds_f);
    auto consume = [&](const Item &it) __attribute__((always_inline)) {
        const float sum = strip_block_sum(it.w, lds, it.table2, it.table3);
        if (it.t < RG) lds_f[geo.value_base + it.t] = half_bits_to_float(it.w[0]) * sum;
    };
    // A wave owns at most 2 PAIRS items (the launcher picks PAIRS from the
    // strip shape), so the loop unrolls completely; the last pair requests
    // nothing after it. Loads are issued whether or not their item is summed.
#pragma unroll
    for (int p = 0; p < PAIRS; ++p) {
        const int j = 2 * p;
        load(item_of(j + 1), wb);
        if (j < n_own) consume(wa);
        if (p + 1 < PAIRS) load(item_of(j + 2), wa);
        if (j + 1 < n_own) consume(wb);
    }
    TQ1_PHASE(strip_wave_id, 3);  // all items summed
    __syncthreads();

    // Row i by the eight lanes 8i .. 8i + 7 (threads 8i + q): lane q adds the
    // values of groups [qG/8, (q + 1)G/8) in group order (-0, the identity of
    // +, for an empty range), then the eight partials are added pairwise
    // across lanes with DPP, ((p0 + p1) + (p2 + p3)) + ((p4 + p5) + (p6 + p7)):
    // quad permutes within each half, then the upper half's sum shifted down
    // four lanes within the row of 16. Lane 8i holds the total. The order is
    // fixed by the shape.
    if (wave < (8 * R + 63) >> 6) {
        const int i = tid >> 3, q = tid & 7;
        float part = -0.0f;
        if (i < R) {
            const float *v = lds_f + geo.value_base + i;
            const int g1 = ((q + 1) * G) >> 3;
            for (int g = (q * G) >> 3; g < g1; ++g) part += v[g * R];
        }
        // DPP: quad_perm [1, 0, 3, 2] swaps neighbours, [2, 3, 0, 1] pairs,
        // row_shl:4 (0x104) reads the lane four above (lanes 12-15 of a row
        // of 16, whose sums are not used, read 0).
        const float pair =
            part + __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(part), 0xb1, 0xf, 0xf, false));
        const float quad =
            pair + __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(pair), 0x4e, 0xf, 0xf, false));
        const float total =
            quad + __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(quad), 0x104, 0xf, 0xf, false));
        if constexpr (GLU) {
            // Rows 2r and 2r + 1 (lo is even) sit eight lanes apart.
            const T own = from_f32<T>(total);
            const float partner = __shfl_xor(to_f32<T>(own), 8, 64);
            if (i < R && (tid & 15) == 0) y[(lo + i) / 2] = swiglu_pair<T>(own, from_f32<T>(partner));
        } else if constexpr (SPLIT) {
            // The Z chunks of a row meet in a fixed binary tree of exchange
            // slots: Z = 2 (c0 + c1), 3 ((c0 + c1) + c2), 4 ((c0 + c1) +
            // (c2 + c3)). At each node a chunk swaps its value into the slot
            // (an agent-scope atomic exchange): finding the slot empty it
            // leaves; finding its sibling's value it adds the two, left child
            // first (two operands: the same sum whichever arrives first),
            // empties the slot and goes on up. The chunk that completes the
            // root stores the row. One atomic round trip per level, nothing to
            // wait for, and the slots are empty again after every call.
            if (i < R && q == 0) {
                unsigned *const row_slots = slots + lo + i;
                const int N = geo.N;
                float v = total;
                auto merge = [&](int node, bool right) __attribute__((always_inline)) {
                    // 0 is an empty slot: values travel as their bits + 1,
                    // NaNs as the quiet NaN (whose bits + 1 is not 0).
                    const uint32_t bits = v != v ? 0x7fc00000u : __float_as_uint(v);
                    const unsigned old = __hip_atomic_exchange(row_slots + static_cast<int64_t>(node) * N, bits + 1u,
                                                               __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    if (old == 0u) return false;
                    const float other = __uint_as_float(old - 1u);
                    v = right ? other + v : v + other;
                    __hip_atomic_store(row_slots + static_cast<int64_t>(node) * N, 0u, __ATOMIC_RELAXED,
                                       __HIP_MEMORY_SCOPE_AGENT);
                    return true;
                };
                bool root;
                if (geo.Z == 2)
                    root = merge(0, z == 1);
                else if (geo.Z == 3)
                    root = (z == 2 || merge(0, z == 1)) && merge(1, z == 2);
                else
                    root = merge(z >> 1, (z & 1) != 0) && merge(2, z >= 2);
                if (root) y[lo + i] = from_f32<T>(v);
            }
        } else {
            if (i < R && q == 0) y[lo + i] = from_f32<T>(total);
        }
    }
    TQ1_PHASE(strip_wave_id, 4);  // done
}

// The elementwise SwiGLU step over a linear's output whose rows alternate
// gate, up: z[i] = SiLU(y[2i]) * y[2i+1] (N even, so pairs never straddle a
// batch row).
template <typename T>
__global__ __launch_bounds__(kThreads) void swiglu_pairs_kernel(const T *__restrict__ y, T *__restrict__ z,
                                                                int64_t pairs) {
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < pairs;
         i += static_cast<int64_t>(gridDim.x) * blockDim.x)
        z[i] = swiglu_pair<T>(y[2 * i], y[2 * i + 1]);
}

template <typename T>
__global__ __launch_bounds__(kThreads) void reduce_partials_kernel(const float *__restrict__ partial,
                                                                   T *__restrict__ y, int64_t count,
                                                                   int splits) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i >= count) return;
    float a = partial[i];
    for (int c = 1; c < splits; ++c) a += partial[static_cast<int64_t>(c) * count + i];
    y[i] = from_f32<T>(a);
}

// ---------------------------------------------------------------------------
// mfma_gemm_kernel: y = x @ W^T on CDNA4 matrix cores.
//
// Workgroup tile 128 (M) x 128 (N), one 128-weight group per K step. Each K
// step stages the activation tile (fp16, straight copy) and decodes the weight
// tile -- 128 rows x one block, read as seven coalesced words per row -- into
// fp16 (t - 1) * scale in LDS (exact in fp16, so the only rounding is the fp32
// accumulation). Four waves in a 2 x 2 grid each own 64 x 64 outputs = 2 x 2
// tiles of v_mfma_f32_32x32x16_f16. LDS rows are padded by 8 halves so the
// 16-byte fragment reads of a wave fall in distinct banks.
// ---------------------------------------------------------------------------
typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float float16v __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((vector_size(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int kGemmBM = 128;
constexpr int kGemmBN = 128;
constexpr int kGemmStride = kBlockWeights + 8;  // halves per LDS row

// Digit carriers: for a byte p <= 242, t = p * 69043 approximates p / 243 in
// 24-bit fixed point and each t = (t mod 2^24) * 3 -- one v_mul_u32_u24,
// which ignores the bits above 24 -- leaves the next base-3 digit, most
// significant first, in bits 24-25 (exact for every legal byte, checked
// exhaustively on the CPU; the tail byte p <= 26 uses 9 * 69043; illegal
// bytes give digits in 0..2). Two carriers become two fp16 weights with two
// v_perm_b32: one gathers their top bytes, the other selects from the table.
using tq1_bytes::byte_digit_carriers;
using tq1_bytes::tail_digit_carriers;

// {-s, z, +s} selected by digit d: selector bytes (2d, 2d+1) per fp16, from a
// pair of carriers' top bytes. z is 0, or NaN when the scale is inf/NaN, so that
// (t - 1) * s keeps IEEE semantics (0 * inf = NaN) exactly.
__device__ __forceinline__ uint32_t weight_pair(uint32_t even, uint32_t odd, uint32_t table_hi, uint32_t table_lo) {
    const uint32_t pair = __builtin_amdgcn_perm(odd, even, 0x0c070c03u);  // top bytes -> bytes 0 and 2
    return __builtin_amdgcn_perm(table_hi, table_lo, __umul24(pair, 0x0202u) + 0x01000100u);
}

__device__ __forceinline__ void scale_tables(uint32_t s, uint32_t &table_hi, uint32_t &table_lo) {
    const uint32_t zero = (s & 0x7c00u) == 0x7c00u ? 0x7e00u : 0u;
    table_lo = (zero << 16) | (s ^ 0x8000u);  // bytes 0-1: -s, bytes 2-3: z
    table_hi = s;                             // bytes 4-5: +s
}

// Decodes weights k = 64H .. 64H+63 of one block, in k order, into 32 dwords
// = 64 fp16 (t - 1) * scale values.
template <int H>
__device__ __forceinline__ void decode_half_block(const uint32_t (&w)[kBlockWords], uint32_t (&out)[32]) {
    uint32_t table_hi, table_lo;
    scale_tables(w[0] & 0xffffu, table_hi, table_lo);
    // Code bytes touched by this half: [first, last]; slot 25 is the tail byte.
    constexpr int first = H == 0 ? 0 : 12;
    constexpr int last = H == 0 ? 12 : kFullSlots;
    uint32_t c[(last - first + 1) * 5];
#pragma unroll
    for (int sl = first; sl <= last; ++sl) {
        const uint32_t p = block_byte(w, 2 + sl);
        uint32_t d[5];
        if (sl < kFullSlots) {
            byte_digit_carriers(p, d);
        } else {
            uint32_t dt[3];
            tail_digit_carriers(p, dt);
            d[0] = dt[0];
            d[1] = dt[1];
            d[2] = dt[2];
            d[3] = d[4] = 0u;
        }
#pragma unroll
        for (int i = 0; i < 5; ++i) c[(sl - first) * 5 + i] = d[i];
    }
#pragma unroll
    for (int p = 0; p < 32; ++p) {
        uint32_t d2[2];
#pragma unroll
        for (int e = 0; e < 2; ++e) {
            const int k = H * 64 + 2 * p + e;
            const int sl = k < 125 ? k / 5 : kFullSlots;
            const int i = k < 125 ? k % 5 : k - 125;
            d2[e] = c[(sl - first) * 5 + i];
        }
        out[p] = weight_pair(d2[0], d2[1], table_hi, table_lo);
    }
}

__global__ __launch_bounds__(kThreads) void mfma_gemm_kernel(
    const uint32_t *__restrict__ packed, const _Float16 *__restrict__ x, _Float16 *__restrict__ y,
    float *__restrict__ partial, int M, int N, int G, int chunk_groups) {
    __shared__ __attribute__((aligned(16))) _Float16 xs[kGemmBM * kGemmStride];
    __shared__ __attribute__((aligned(16))) _Float16 ws[kGemmBN * kGemmStride];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int n0 = blockIdx.x * kGemmBN;
    const int m0 = blockIdx.y * kGemmBM;
    const int chunk = blockIdx.z;
    const int g_begin = chunk * chunk_groups;
    const int g_end = min(G, g_begin + chunk_groups);
    const int64_t K = static_cast<int64_t>(G) * kBlockWeights;
    const int wm = (wave >> 1) * 64;
    const int wn = (wave & 1) * 64;

    float16v acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

    // Decoder assignment: lanes own consecutive rows (coalesced word loads);
    // rows past N decode the last row and their tile rows are never stored.
    const int dec_row = tid & (kGemmBN - 1);
    const int dec_half = tid / kGemmBN;
    const int dec_n = min(n0 + dec_row, N - 1);
    const uint32_t *dec_words =
        packed + static_cast<int64_t>(dec_n / kTileRows) * G * kTileGroupWords + (dec_n % kTileRows);
    // Activation assignment: 128 rows x 16 chunks of 8 halves, 8 per thread;
    // rows past M read row M-1 and are never stored.
    const _Float16 *x_rows[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const int idx = tid + i * kThreads;
        x_rows[i] = x + static_cast<int64_t>(min(m0 + (idx >> 4), M - 1)) * K + (idx & 15) * 8;
    }

    // Prefetch the first group.
    half8 xv[8];
    uint32_t wv[kBlockWords];
#pragma unroll
    for (int i = 0; i < 8; ++i)
        xv[i] = *reinterpret_cast<const half8 *>(x_rows[i] + static_cast<int64_t>(g_begin) * kBlockWeights);
#pragma unroll
    for (int j = 0; j < kBlockWords; ++j) wv[j] = dec_words[static_cast<int64_t>(g_begin) * kTileGroupWords + j * kTileRows];

    for (int g = g_begin; g < g_end; ++g) {
        // Stage this group: activations as loaded, weights decoded.
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const int idx = tid + i * kThreads;
            *reinterpret_cast<half8 *>(xs + (idx >> 4) * kGemmStride + (idx & 15) * 8) = xv[i];
        }
        {
            uint32_t dec[32];
            if (dec_half == 0)
                decode_half_block<0>(wv, dec);
            else
                decode_half_block<1>(wv, dec);
#pragma unroll
            for (int q = 0; q < 8; ++q) {
                uint4 v = {dec[4 * q], dec[4 * q + 1], dec[4 * q + 2], dec[4 * q + 3]};
                *reinterpret_cast<uint4 *>(ws + dec_row * kGemmStride + dec_half * 64 + q * 8) = v;
            }
        }
        __syncthreads();
        // Next group's operands are in flight during this group's MFMAs.
        if (g + 1 < g_end) {
#pragma unroll
            for (int i = 0; i < 8; ++i)
                xv[i] = *reinterpret_cast<const half8 *>(x_rows[i] + static_cast<int64_t>(g + 1) * kBlockWeights);
#pragma unroll
            for (int j = 0; j < kBlockWords; ++j)
                wv[j] = dec_words[static_cast<int64_t>(g + 1) * kTileGroupWords + j * kTileRows];
        }
#pragma unroll
        for (int kk = 0; kk < kBlockWeights / 16; ++kk) {
            half8 a[2], b[2];
            const int kofs = kk * 16 + (lane >> 5) * 8;
#pragma unroll
            for (int i = 0; i < 2; ++i)
                a[i] = *reinterpret_cast<const half8 *>(xs + (wm + i * 32 + (lane & 31)) * kGemmStride + kofs);
#pragma unroll
            for (int j = 0; j < 2; ++j)
                b[j] = *reinterpret_cast<const half8 *>(ws + (wn + j * 32 + (lane & 31)) * kGemmStride + kofs);
#pragma unroll
            for (int i = 0; i < 2; ++i)
#pragma unroll
                for (int j = 0; j < 2; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a[i], b[j], acc[i][j], 0, 0, 0);
        }
        __syncthreads();
    }

    // D[i][j] of a 32x32 tile sits in lane j + 32 * ((i / 4) % 2), item 4 * (i / 8) + i % 4.
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int m = m0 + wm + i * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
                const int n = n0 + wn + j * 32 + (lane & 31);
                if (m < M && n < N) {
                    if (partial)
                        partial[(static_cast<int64_t>(chunk) * M + m) * N + n] = acc[i][j][r];
                    else
                        y[static_cast<int64_t>(m) * N + n] = static_cast<_Float16>(acc[i][j][r]);
                }
            }
}

// ---------------------------------------------------------------------------
// direct_gemm_kernel: the "direct fragments" form for small batches (M <= 64).
//
// Weights never touch LDS: each lane decodes half of one block straight into
// the A operand of v_mfma_f32_32x32x16_f16 (weight rows x K); the activations
// are the B operand (K x batch). A workgroup (4 waves, 128 weight rows) copies
// a window of its K chunk's activations into LDS (through registers for up to
// 16 rows, by LDS-DMA for more), then each wave runs the window's groups with
// no barrier: a wave owns 32 weight rows, lane l decodes half h = l / 32 of
// row l % 32's block and reads 5 of the block's 7 words. NB = ceil(M / 32)
// tiles.
//
// K order. The dot product over a group does not depend on the order of its
// 128 terms, so both operands use one fixed permutation that makes the two
// halves decode with the same code: half h takes code bytes 12h .. 12h+11
// (trits 60h .. 60h+59) as positions 0..59, then positions 60..63 are trits
// 120..123 (digits 0-3 of code byte 24) for h = 0, and trits 124..127 (digit 4
// of code byte 24, the three tail trits) for h = 1. MFMA step s takes positions
// 8s .. 8s+7 of half h as its K slice 16s + 8h. The activation rows are staged
// in that order: logical 4-half unit u holds physical unit u (u < 15), 30
// (u = 15), u - 1 (16 <= u < 31) or 31 (u = 31).
//
// Weights. A lane turns its half block into 32 dwords of fp16 weight pairs:
// each pair of code bytes is split two bytes per 16-bit-packed operation and
// indexes six small selector tables in LDS (tq1_bytes.h, half_block_selectors
// below), and one v_perm_b32 per pair selects the pair's two fp16 values from
// {-s, z, +s} (z is 0, or NaN for a non-finite scale, as (t - 1) * s gives).
// Every byte value, legal or not, indexes inside the tables (checked on the
// CPU over all of them). The wide form decodes the same way; the LDS-tile
// form keeps the 24-bit digit carriers of tq1_bytes.h.
// ---------------------------------------------------------------------------
constexpr int kBufferRsrcFlags = 0x00020000;  // gfx9 raw buffer resource: 32-bit data format
constexpr int kDirectWaves = 4;
constexpr int kDirectThreads = kDirectWaves * 64;
constexpr int kDirectRows = kDirectWaves * 32;          // weight rows per workgroup
constexpr int kDirectLdsBytes = 160 * 1024 - 1024;      // dynamic LDS budget (gfx950: 160 KiB per workgroup)
constexpr int kDirectStride = kBlockWeights + 8;      // halves per staged activation row


// The 32 selector dwords of one half block (pairs of weights, in the direct K
// order), from the selector tables in LDS (sel_bytes, tq1_bytes.h): u[0..3]
// hold the half's twelve code bytes at bytes 2..13, w6 code byte 24 (byte 2)
// and the tail byte (byte 3). Code bytes 2w, 2w+1 (window w) give pairs
// 5w .. 5w+4; pairs 30 and 31 are code byte 24's first four weights in the
// lower half and, in the upper half, its fifth with the three tail weights.
// The work comes in pieces that a caller can spread over its MFMA stages: the
// split of windows 2k and 2k+1 (window_splits, VALU only), the five table
// reads of one window (window_selectors) and the tail's (tail_selectors).
// Selectors 5w+2 and 30 are the OR of two table reads; the pieces leave the
// second in late[w] (late[6] for selector 30), for the consumer to OR in where
// it takes the selector, rather than wait for the reads it has just issued.
struct WindowSplits {
    uint32_t la, ha, lb, hb;  // a / 9, a % 9, b / 27, b % 27 of both windows, one per 16-bit half
};

__device__ __forceinline__ WindowSplits window_splits(const uint32_t (&u)[4], int k) {
    // the a bytes (even code bytes) of windows 2k, 2k+1 and their b bytes,
    // one per 16-bit half
    const u16x2 a = __builtin_bit_cast(u16x2, __builtin_amdgcn_perm(u[k + 1], u[k], 0x0c040c02u));
    const u16x2 b = __builtin_bit_cast(u16x2, __builtin_amdgcn_perm(u[k + 1], u[k], 0x0c050c03u));
    const u16x2 ha = tq1_bytes::lut23_high(a), la = tq1_bytes::lut23_low(a, ha);
    const u16x2 hb = tq1_bytes::split27_high(b), lb = tq1_bytes::split27_low(b, hb);
    return WindowSplits{__builtin_bit_cast(uint32_t, la), __builtin_bit_cast(uint32_t, ha),
                        __builtin_bit_cast(uint32_t, lb), __builtin_bit_cast(uint32_t, hb)};
}

__device__ __forceinline__ uint32_t selector_lds(const char *sel_bytes, uint32_t address, int entry) {
    return *reinterpret_cast<const uint32_t *>(sel_bytes + address + entry * 4);
}

// Window 2k + e of splits s (window_splits(u, k)): selectors 5w .. 5w+4.
__device__ __forceinline__ void window_selectors(const WindowSplits &s, int k, int e, const char *sel_bytes,
                                                 uint32_t (&sel)[32], uint32_t (&late)[7]) {
    const uint32_t zero = 0;
    const int w = 2 * k + e;
    const uint32_t al = e ? lut_address_hi(s.la, zero) : lut_address_lo(s.la, zero);
    const uint32_t ah = e ? lut_address_hi(s.ha, zero) : lut_address_lo(s.ha, zero);
    const uint32_t bl = e ? lut_address_hi(s.lb, zero) : lut_address_lo(s.lb, zero);
    const uint32_t bh = e ? lut_address_hi(s.hb, zero) : lut_address_lo(s.hb, zero);
    sel[5 * w] = selector_lds(sel_bytes, al, tq1_bytes::kSelT9a);
    sel[5 * w + 1] = selector_lds(sel_bytes, ah, tq1_bytes::kSelT27aX);
    sel[5 * w + 2] = selector_lds(sel_bytes, ah, tq1_bytes::kSelT27aY);
    late[w] = selector_lds(sel_bytes, bl, tq1_bytes::kSelT27bX);
    sel[5 * w + 3] = selector_lds(sel_bytes, bl, tq1_bytes::kSelT27bY);
    sel[5 * w + 4] = selector_lds(sel_bytes, bh, tq1_bytes::kSelT9b);
}

// Selectors 30 and 31 from code byte 24 and the tail byte (w6).
__device__ __forceinline__ void tail_selectors(uint32_t w6, bool upper, const char *sel_bytes, uint32_t (&sel)[32],
                                               uint32_t (&late)[7]) {
    // (The half-dependent choices as bit blends with a lane mask: written as
    // selects, they became an exec-masked branch.)
    const uint32_t mask = 0u - static_cast<uint32_t>(upper);
    auto blend = [&](uint32_t if_upper, uint32_t if_lower) { return (if_upper & mask) | (if_lower & ~mask); };
    const uint32_t p24 = (w6 >> 16) & 0xffu;
    const uint32_t t = tq1_bytes::tail_entry(w6 >> 24);
    const uint32_t h24 = (p24 * 57u) >> 9, l24 = p24 - 9u * h24;
    const uint32_t lead =
        selector_lds(sel_bytes, blend(4 * (t + tq1_bytes::kSelT27bX), 4 * (l24 + tq1_bytes::kSelT9a)), 0);
    const uint32_t rest =
        selector_lds(sel_bytes, blend(4 * (t + tq1_bytes::kSelT27bY), 4 * (h24 + tq1_bytes::kSelT27aX)), 0);
    const uint32_t fifth = selector_lds(sel_bytes, 4 * h24, tq1_bytes::kSelT27aY);
    sel[30] = lead;
    late[6] = fifth & mask;
    sel[31] = rest;
}

// Selector q with its late part (see above).
__device__ __forceinline__ uint32_t full_selector(const uint32_t (&sel)[32], const uint32_t (&late)[7], int q) {
    return q == 30 ? sel[30] | late[6] : (q < 30 && q % 5 == 2 ? sel[q] | late[q / 5] : sel[q]);
}

__device__ __forceinline__ void half_block_selectors(const uint32_t (&u)[4], uint32_t w6, bool upper,
                                                     const char *sel_bytes, uint32_t (&sel)[32]) {
    uint32_t late[7];
#pragma unroll
    for (int k = 0; k < 3; ++k) {
        const WindowSplits s = window_splits(u, k);
#pragma unroll
        for (int e = 0; e < 2; ++e) {
            window_selectors(s, k, e, sel_bytes, sel, late);
            sel[5 * (2 * k + e) + 2] |= late[2 * k + e];
        }
    }
    tail_selectors(w6, upper, sel_bytes, sel, late);
    sel[30] |= late[6];
}

// One pipeline step of direct_gemm_kernel: the MFMAs of the current group
// (weights already decoded in a_mfma, activations in LDS buffer `buf`) with the
// decode of the next group (words u, other -> a_dec): its 32 selector dwords
// from the tables in LDS up front, then at stage st the four weight pairs MFMA
// step st of the following group will need.
template <int NB, bool kMfma = true>
__device__ __forceinline__ void direct_step(float16v (&acc)[NB], const uint32_t (&a_mfma)[32], uint32_t (&a_dec)[32],
                                            const uint32_t (&u)[4], uint32_t other, bool upper,
                                            const _Float16 *xb, const char *sel_bytes,
                                            uint32_t scale_mask = 0xffffu) {
    // scale_mask 0 turns a padding group's weights into +-0.
    uint32_t table_hi, table_lo;
    scale_tables((upper ? other : u[0]) & scale_mask, table_hi, table_lo);
    uint32_t sel[32];
#pragma unroll
    for (int st = 0; st < 8; ++st) {
        half8 bf[NB];
#pragma unroll
        for (int nb = 0; nb < NB; ++nb)
            bf[nb] = *reinterpret_cast<const half8 *>(xb + nb * 32 * kDirectStride + st * 8);
        if (st == 0) half_block_selectors(u, upper ? u[3] : other, upper, sel_bytes, sel);
#pragma unroll
        for (int p = 4 * st; p < 4 * st + 4; ++p) a_dec[p] = __builtin_amdgcn_perm(table_hi, table_lo, sel[p]);
        if (!kMfma) continue;
        half8 af;
        {
            uint4 v = {a_mfma[4 * st], a_mfma[4 * st + 1], a_mfma[4 * st + 2], a_mfma[4 * st + 3]};
            af = *reinterpret_cast<half8 *>(&v);
        }
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) acc[nb] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af, bf[nb], acc[nb], 0, 0, 0);
    }
}

// MFMA steps of one group with weights already decoded (no decode).
template <int NB>
__device__ __forceinline__ void direct_mfma(float16v (&acc)[NB], const uint32_t (&a)[32], const _Float16 *xb) {
#pragma unroll
    for (int st = 0; st < 8; ++st) {
        half8 af;
        {
            uint4 v = {a[4 * st], a[4 * st + 1], a[4 * st + 2], a[4 * st + 3]};
            af = *reinterpret_cast<half8 *>(&v);
        }
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) {
            const half8 bf = *reinterpret_cast<const half8 *>(xb + nb * 32 * kDirectStride + st * 8);
            acc[nb] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af, bf, acc[nb], 0, 0, 0);
        }
    }
}

// Logical 4-half unit u of a staged activation row holds physical unit
// direct_source_unit(u) of the group (the K order above).
__device__ __forceinline__ int direct_source_unit(int u) { return u < 15 ? u : (u == 15 ? 30 : (u < 31 ? u - 1 : 31)); }

// Three waves per SIMD (168 VGPRs at most; the two-tile form keeps one 8-byte
// value in scratch, reloaded once per eight-group loop pass): a CU then holds
// three workgroups, so the grid (about 2.7 workgroups per CU at the 27B
// shapes) runs in one round.
template <int NB, int SR>
__global__ __launch_bounds__(kDirectThreads, 3) void direct_gemm_kernel(
    const uint32_t *__restrict__ packed, const _Float16 *__restrict__ x, _Float16 *__restrict__ y,
    float *__restrict__ partial, unsigned *__restrict__ counters, int M, int N, int G, int chunk_groups,
    int k_split, int window) {
    static_assert(SR <= 32 * NB && SR >= 8, "staged rows");
    extern __shared__ __attribute__((aligned(16))) _Float16 xs[];  // window x SR rows x kDirectStride halves
    __shared__ unsigned s_last;
    __shared__ uint32_t selectors[tq1_bytes::kSelEntries];

    const int tid = threadIdx.x;
    if (tid < tq1_bytes::kSelEntries) selectors[tid] = tq1_bytes::selector_entry(tid);  // read after the first barrier
    const char *const sel_bytes = reinterpret_cast<const char *>(selectors);
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // uniform: LDS-DMA bases go in M0
    const bool upper = lane >= 32;
    const int row0 = blockIdx.x * kDirectRows + wave * 32;
    const int g_begin = blockIdx.y * chunk_groups;
    const int cg = chunk_groups;
    const int direct_wave_id = (blockIdx.y * gridDim.x + blockIdx.x) * kDirectWaves + wave;
    (void)direct_wave_id;
    TQ1_PHASE(direct_wave_id, 0);  // wave start
    TQ1_PHASE_XCC(direct_wave_id);
    const int64_t K = static_cast<int64_t>(G) * kBlockWeights;

    // Rows past the padded last tile load the last padded row (discarded).
    const int load_row = min(row0 + (lane & 31), ceil_div_dev(N, kTileRows) * kTileRows - 1);
    const uint32_t *wrow = packed + static_cast<int64_t>(load_row / kTileRows) * G * kTileGroupWords + (load_row % kTileRows);
    const int wfirst = (upper ? 3 : 0) * kTileRows;
    const int wother = (upper ? 0 : 6) * kTileRows;
    const int src_half = direct_source_unit(lane >> 1) * 4 + (lane & 1) * 2;

    // B fragments: activation row (lane & 31) (+32 for the second tile); rows
    // past SR read row SR - 1 (their MFMA columns are never stored).
    const int brow = min(lane & 31, SR - 1);
    const int bofs = brow * kDirectStride + (upper ? 64 : 0);

    float16v acc[NB];
#pragma unroll
    for (int nb = 0; nb < NB; ++nb)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[nb][r] = 0.0f;

    constexpr int CH = 4;  // groups of words per prefetch set
    for (int w0 = 0; w0 < cg; w0 += window) {
        const int wn = min(window, cg - w0);
        const int gw = g_begin + w0;
        auto load_chunk = [&](uint32_t (&w)[CH][5], int q) {
#pragma unroll
            for (int c = 0; c < CH; ++c) {
                const uint32_t *p = wrow + static_cast<int64_t>(gw + min(q + c, wn - 1)) * kTileGroupWords;
#pragma unroll
                for (int j = 0; j < 4; ++j) w[c][j] = p[wfirst + j * kTileRows];
                w[c][4] = p[wother];
            }
        };
        auto xb = [&](int q) { return xs + q * SR * kDirectStride + bofs; };

        if (w0) __syncthreads();  // every wave is done with the previous window's activations
        // The window's activations, staged in LDS in the K order above
        // (logical unit u of a row, 4 halves, from physical unit
        // direct_source_unit(u); rows past M re-read row M - 1). Up to 16
        // staged rows, 32 rows in windows of up to 4 groups and 64 in windows
        // of up to 2 (the planner's windows there): as 16-byte physical chunks
        // loaded into registers (8 per thread at 16 rows x 8 groups, 32 x 4 or
        // 64 x 2) ahead of the first word set, each written to LDS after it
        // as two 8-byte units at their K-order positions -- loads complete in
        // order, so the writes wait for the activations only while the words
        // are in flight. Otherwise by LDS-DMA (one padded row per instruction)
        // waited for before any word is requested, as a second register pass
        // would wait for the words too. The second word set is requested after
        // the staging barrier, so no wave reaches the barrier late for issuing
        // it behind the CU's memory queue (M=8-32, every 27B shape, 1-3 %
        // faster on MI355X). (Measured on MI355X, gate/up: M=16 20.7 -> 19.0
        // us and M=8 19.2 -> 18.3 us with 8-byte units in registers, 17.1 us
        // at M=8 with 16-byte chunks; M=32 in 8-group windows 27.8 us with
        // LDS-DMA against 32.4 with registers, 20.3 us in 4-group windows with
        // registers.)
        uint32_t wa[CH][5], wb[CH][5];
        if (SR <= 16 || wn * SR * 16 <= 8 * kDirectThreads) {
            constexpr int kUnits = 16;  // per thread
            const int units = wn * SR * 32;
            auto unit_source = [&](int i) {
                const int r = i >> 5, q = r / SR, m = r - q * SR;
                return reinterpret_cast<const uint2 *>(x + static_cast<int64_t>(min(m, M - 1)) * K +
                                                       static_cast<int64_t>(gw + q) * kBlockWeights +
                                                       direct_source_unit(i & 31) * 4);
            };
            auto unit_target = [&](int i) {
                return reinterpret_cast<uint2 *>(xs + (i >> 5) * kDirectStride + (i & 31) * 4);
            };
            // Indices past the window are clamped (those threads load and write
            // the last unit again, the same value): no load or write behind a
            // branch, where the compiler's wait counts turn conservative.
            const int first = min(units, kUnits * kDirectThreads);
            // 16-byte physical chunks: chunk j is row-group j / 16, physical
            // units 2 (j % 16) and 2 (j % 16) + 1, written to their K-order
            // positions (the inverse of direct_source_unit).
            auto target_unit = [](int u) { return u < 15 ? u : (u < 30 ? u + 1 : (u == 30 ? 15 : 31)); };
            const int first_chunks = first / 2;
            uint4 xc[kUnits / 2];
#pragma unroll
            for (int k = 0; k < kUnits / 2; ++k) {
                const int j = min(tid + k * kDirectThreads, first_chunks - 1);
                const int r = j >> 4, q = r / SR, m = r - q * SR;
                xc[k] = *reinterpret_cast<const uint4 *>(x + static_cast<int64_t>(min(m, M - 1)) * K +
                                                         static_cast<int64_t>(gw + q) * kBlockWeights + (j & 15) * 8);
            }
            __builtin_amdgcn_sched_barrier(0);
            load_chunk(wa, 0);
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int k = 0; k < kUnits / 2; ++k) {
                const int j = min(tid + k * kDirectThreads, first_chunks - 1);
                const int r = j >> 4, c = j & 15;
                *reinterpret_cast<uint2 *>(xs + r * kDirectStride + target_unit(2 * c) * 4) = uint2{xc[k].x, xc[k].y};
                *reinterpret_cast<uint2 *>(xs + r * kDirectStride + target_unit(2 * c + 1) * 4) = uint2{xc[k].z, xc[k].w};
            }
            // (Windows of more than 8 groups at 16 rows: the rest after the words.)
            for (int i = first + tid; i < units; i += kDirectThreads) *unit_target(i) = *unit_source(i);
        } else {
            for (int r = wave; r < wn * SR; r += kDirectWaves) {
                const int q = r / SR, m = r - q * SR;
                const _Float16 *src = x + static_cast<int64_t>(min(m, M - 1)) * K +
                                      static_cast<int64_t>(gw + q) * kBlockWeights + src_half;
                __builtin_amdgcn_global_load_lds((const __attribute__((address_space(1))) void *)src,
                                                 (__attribute__((address_space(3))) void *)(xs + r * kDirectStride),
                                                 4, 0, 0);
            }
            wait_vector_memory();
            load_chunk(wa, 0);
        }
        if (w0 == 0) TQ1_PHASE(direct_wave_id, 1);  // first window's activations staged
        __syncthreads();
        __builtin_amdgcn_sched_barrier(0);
        load_chunk(wb, CH);
        __builtin_amdgcn_sched_barrier(0);

        // Pipeline over the window (no barriers): MFMAs of group q interleaved
        // with the decode of q+1; words come in sets of four groups issued four
        // steps before their first decode. Decoded weights alternate with
        // period 2 and word sets with period 8, so the loop body is 8 steps and
        // no register is copied (a copy would wait for its prefetch).
        uint32_t a0[32], a1[32];
        {
            const uint32_t u[4] = {wa[0][0], wa[0][1], wa[0][2], wa[0][3]};
            direct_step<NB, false>(acc, a1, a0, u, wa[0][4], upper, xb(0), sel_bytes);
        }
        auto step = [&](const uint32_t (&a_mfma)[32], uint32_t (&a_dec)[32], const uint32_t (&w)[5], int q) {
            const uint32_t u[4] = {w[0], w[1], w[2], w[3]};
            direct_step<NB>(acc, a_mfma, a_dec, u, w[4], upper, xb(q), sel_bytes);
        };
        int q = 0;
        for (; q + 2 * CH <= wn; q += 2 * CH) {
            step(a0, a1, wa[1], q + 0);
            step(a1, a0, wa[2], q + 1);
            step(a0, a1, wa[3], q + 2);
            step(a1, a0, wb[0], q + 3);
            // The fences keep the scheduler from sinking the prefetch toward its use.
            __builtin_amdgcn_sched_barrier(0);
            load_chunk(wa, q + 2 * CH);
            __builtin_amdgcn_sched_barrier(0);
            step(a0, a1, wb[1], q + 4);
            step(a1, a0, wb[2], q + 5);
            step(a0, a1, wb[3], q + 6);
            step(a1, a0, wa[0], q + 7);
            __builtin_amdgcn_sched_barrier(0);
            load_chunk(wb, q + 3 * CH);
            __builtin_amdgcn_sched_barrier(0);
        }
        // Four groups left (a window of 4 or 8k + 4 groups): a0 holds group q
        // decoded and wa the words of groups q .. q+3 -- prefetched by the
        // loop above or, for a 4-group window, before it -- so they run the
        // same pipeline.
        if (wn - q == CH) {
            step(a0, a1, wa[1], q + 0);
            step(a1, a0, wa[2], q + 1);
            step(a0, a1, wa[3], q + 2);
            direct_mfma<NB>(acc, a1, xb(q + 3));
            q += CH;
        }
        // Other remainders: a0 holds group q decoded; the next group's words
        // are loaded where they are needed.
        for (; q < wn; ++q) {
            direct_mfma<NB>(acc, a0, xb(q));
            if (q + 1 < wn) {
                const uint32_t *p = wrow + static_cast<int64_t>(gw + q + 1) * kTileGroupWords;
                const uint32_t u[4] = {p[wfirst], p[wfirst + kTileRows], p[wfirst + 2 * kTileRows], p[wfirst + 3 * kTileRows]};
                direct_step<NB, false>(acc, a1, a0, u, p[wother], upper, xb(q + 1), sel_bytes);
            }
        }
    }

    TQ1_PHASE(direct_wave_id, 5);  // every group summed
    // D[i][j] of a 32x32 tile sits in lane j + 32 * ((i / 4) % 2), item 4 * (i / 8) + i % 4;
    // here i is a weight row of the wave and j an activation row.
    if (k_split > 1) {
        // Partials in quads, only the lanes of real activation rows: values
        // 4q .. 4q+3 of tile nb in lane j + 32 h (j < S = min(M, 32)) sit at
        // ((nb * 4 + q) * 2 S + h * S + j) * 4 of the (chunk, wave) region, so
        // a lane stores and loads them with four 16-byte device-coherent (sc1)
        // buffer accesses, each instruction covering 2 S * 16 contiguous bytes.
        // The chunk, tile and quad offsets are wave-uniform (scalar).
        constexpr int kDeviceCoherent = 16;  // cache policy SC1
        const int S = min(M, 32);
        const int frag = NB * 32 * S;
        const int64_t chunk_stride = static_cast<int64_t>(kDirectWaves) * frag;
        const int j = lane & 31;
        const float *wave_base = partial + static_cast<int64_t>(blockIdx.x) * k_split * chunk_stride +
                                 static_cast<int64_t>(wave) * frag;
        const __amdgpu_buffer_rsrc_t rp = __builtin_amdgcn_make_buffer_rsrc(
            const_cast<float *>(wave_base), 0, static_cast<int>(k_split * chunk_stride * 4), kBufferRsrcFlags);
        // lanes past the real rows load row S - 1 again (never stored)
        const uint32_t voff = static_cast<uint32_t>(((lane >> 5) * S + min(j, S - 1)) * 16);
        auto value_offset = [&](int z, int nb, int q) {
            return static_cast<int>((z * chunk_stride + (nb * 4 + q) * 2 * S * 4) * 4);
        };
#pragma unroll
        for (int nb = 0; nb < NB; ++nb)
            if (nb * 32 + j < M)
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const f32x4 v4 = {acc[nb][4 * q], acc[nb][4 * q + 1], acc[nb][4 * q + 2], acc[nb][4 * q + 3]};
                    __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, v4), rp, voff,
                                                           value_offset(blockIdx.y, nb, q), kDeviceCoherent);
                }
        // Every store acknowledged at the coherence point before the arrival
        // is counted; the compiler barriers keep the stores above the wait.
        asm volatile("" ::: "memory");
        wait_vector_memory();
        asm volatile("" ::: "memory");
        TQ1_PHASE(direct_wave_id, 6);  // partial stored and acknowledged
        __syncthreads();
        unsigned *counter = counters + blockIdx.x;
        if (tid == 0)
            s_last = __hip_atomic_fetch_add(counter, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
                     static_cast<unsigned>(k_split - 1);
        __syncthreads();
        TQ1_PHASE(direct_wave_id, 7);  // arrival counted
        if (!s_last) return;
#pragma unroll
        for (int nb = 0; nb < NB; ++nb)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[nb][r] = 0.0f;
        // The chunks are added in chunk order, all loads of a batch issued
        // before its first add (a batch past the last chunk re-reads it and
        // adds nothing): one tile and up to 8 chunks in one batch; more chunks
        // (down: 17) one half of the 16 values at a time with up to 17 chunks
        // of it per batch, 34 loads in flight; two tiles 4 chunks per batch.
        auto load4 = [&](int z, int nb, int q) {
            return __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                                 rp, voff, value_offset(min(z, k_split - 1), nb, q),
                                                 kDeviceCoherent));
        };
        if (NB == 1 && k_split > 8) {
            constexpr int kHalfBatch = 17;
            for (int z0 = 0; z0 < k_split; z0 += kHalfBatch) {
#pragma unroll
                for (int h = 0; h < 2; ++h) {
                    f32x4 v[kHalfBatch][2];
#pragma unroll
                    for (int u = 0; u < kHalfBatch; ++u)
#pragma unroll
                        for (int q = 0; q < 2; ++q) v[u][q] = load4(z0 + u, 0, 2 * h + q);
#pragma unroll
                    for (int u = 0; u < kHalfBatch; ++u)
                        if (z0 + u < k_split)
#pragma unroll
                            for (int q = 0; q < 2; ++q)
#pragma unroll
                                for (int e = 0; e < 4; ++e) acc[0][8 * h + 4 * q + e] += v[u][q][e];
                }
            }
        } else {
            constexpr int kBatch = NB == 1 ? 8 : 4;
            for (int z0 = 0; z0 < k_split; z0 += kBatch) {
                f32x4 v[kBatch][NB][4];
#pragma unroll
                for (int u = 0; u < kBatch; ++u)
#pragma unroll
                    for (int nb = 0; nb < NB; ++nb)
#pragma unroll
                        for (int q = 0; q < 4; ++q) v[u][nb][q] = load4(z0 + u, nb, q);
#pragma unroll
                for (int u = 0; u < kBatch; ++u)
                    if (z0 + u < k_split)
#pragma unroll
                        for (int nb = 0; nb < NB; ++nb)
#pragma unroll
                            for (int q = 0; q < 4; ++q)
#pragma unroll
                                for (int e = 0; e < 4; ++e) acc[nb][4 * q + e] += v[u][nb][q][e];
            }
        }
        if (tid == 0) __hip_atomic_store(counter, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        TQ1_PHASE(direct_wave_id, 8);  // fix-up sums done
    }
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) {
        const int m = nb * 32 + (lane & 31);
        if (m >= M) continue;
        _Float16 *yrow = y + static_cast<int64_t>(m) * N;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const int n = row0 + 8 * q + 4 * (lane >> 5);
#pragma unroll
            for (int e = 0; e < 4; ++e)
                if (n + e < N) yrow[n + e] = static_cast<_Float16>(acc[nb][4 * q + e]);
        }
    }
}

// ---------------------------------------------------------------------------
// wide_gemm_kernel: prefill y = x @ W^T (large M), direct fragments at scale.
//
// Tile = 256 weight rows x 256 activation rows; a workgroup of 8 waves, two
// per SIMD, so that the trit decode (VALU) of one wave issues while the other
// wave's MFMAs run. Wave w owns weight rows 32w .. 32w+31: lane l decodes half
// l/32 of the block of row l%32 (the direct form's K order) straight into the
// A operand, and each A operand feeds the 8 MFMAs of the tile's 32-row
// activation blocks, so a decoded dword serves 8 MFMAs.
//
// Both operands reach LDS by DMA through buffer resources (no address VALU in
// the loop; rows past the end of x or of the packed array read as zero): per
// group step a 64 KiB activation tile and the tile's 7 KiB of packed words, in
// two-deep rings. At step u the activations of u+1 and the words of u+2 are
// issued, the words of u+1 are read and decoded stage by stage between the
// MFMAs of u (over the A registers each stage has just consumed), and the step
// ends with vmcnt(0) and a barrier: one step of MFMAs hides the DMA latency.
//
// Work is split stream-K: the (tile, group) units, tiles ordered activation
// block major, are cut into gridDim.x equal contiguous ranges, one per
// workgroup, so every CU gets the same number of group steps whatever the
// tile count. A tile a workgroup covers completely is written directly; a
// boundary segment is stored as an fp32 partial (slot 0 = the workgroup's
// first segment, slot 1 = its last), and the last contributor to arrive adds
// the tile's partials in workgroup order (deterministic) and writes it.
// ---------------------------------------------------------------------------
constexpr int kWideWaves = 8;
constexpr int kWideThreads = kWideWaves * 64;
constexpr int kWideRows = kWideWaves * 32;                 // weight rows per tile
constexpr int kWideMaxBlocks = 8;                          // 32-row activation blocks per tile, at most
constexpr int kWideMaxCols = kWideMaxBlocks * 32;          // activation rows per tile, at most
constexpr int kWideRowBlocks = kWideRows / kTileRows;      // 64-row packed blocks per tile
constexpr int kWideWBytes = kWideRowBlocks * kTileGroupWords * 4;  // one group of a tile's words
// Per template width NB (32-row activation blocks per tile): one group of a
// tile's activations, the dynamic LDS, one wave's accumulators.
constexpr int wide_x_bytes(int nb) { return nb * 32 * kBlockWeights * 2; }
// DMA ring depth (units): four where 160 KiB of LDS hold it, so that the
// prefetch distance covers the memory latency when a step is short (narrow
// tiles; measured on MI355X, two workgroups per CU with shallower rings were
// slower at M = 8 and 64).
constexpr int wide_ring(int nb) { return nb >= 8 ? 2 : 4; }
constexpr size_t wide_lds_bytes(int nb) {
    return wide_ring(nb) * (static_cast<size_t>(wide_x_bytes(nb)) + kWideWBytes);
}
constexpr int wide_frag_floats(int nb) { return nb * 16 * 64; }
constexpr int kWideTileSlots = 8184;                       // stream-K counter pairs (arrivals, publications)
constexpr int kXcds = 8;                                   // MI355X: 8 XCDs of 32 CUs, each with its own L2


struct WideGeometry {
    int M, N, G;
    int row_blocks;  // ceil(N / 64)
    int tiles_n;     // weight row blocks of 256
    int tiles;       // tiles_n * ceil(M / (32 NB))
    int units;       // tiles * G
    int vector_rows; // y rows start 16-byte aligned (y aligned, N % 8 == 0)
    int spin_limit;  // polls of the publication count before the last arriver gives up
};


// Units are counted in 32 bits: at most 16384 tiles x 32768 groups.
__device__ __forceinline__ int wide_unit_begin(int units, int p, int P) {
    return static_cast<int>(static_cast<int64_t>(units) * p / P);
}
__device__ __forceinline__ int wide_owner(int units, int u, int P) {
    return static_cast<int>((static_cast<int64_t>(u + 1) * P - 1) / units);
}

// Activations in the direct forms' K order: within every group, 4-half unit u
// of the copy is unit direct_source_unit(u) of x, so that the wide kernel can
// stage 16-byte runs with LDS-DMA.
// A thread writes four consecutive units of the copy (two 16-byte stores when
// the copy is 16-byte aligned): a quarter of the threads and half of the store
// instructions of a unit-per-thread copy.
__global__ __launch_bounds__(kThreads) void permute_activations_kernel(const uint2 *__restrict__ x,
                                                                      uint2 *__restrict__ xp, int64_t quads,
                                                                      int wide_stores) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
    if (i >= quads) return;
    const int64_t base = (i >> 3) * 32;  // the group's first unit
    const int u0 = static_cast<int>(i & 7) * 4;
    uint2 v[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) v[k] = x[base + direct_source_unit(u0 + k)];
    if (wide_stores) {
        uint4 *dst = reinterpret_cast<uint4 *>(xp + base + u0);
        dst[0] = uint4{v[0].x, v[0].y, v[1].x, v[1].y};
        dst[1] = uint4{v[2].x, v[2].y, v[3].x, v[3].y};
    } else {
#pragma unroll
        for (int k = 0; k < 4; ++k) xp[base + u0 + k] = v[k];
    }
}

// bf16 activations for the wide form: one workgroup per activation row. The
// row's largest finite magnitude sets a power of two s that puts it in
// [2^14, 2^15); the copy holds fp16(x s), in the wide form's K order when
// PERMUTE (the permuted copy above), and inv[m] = 1 / s. The conversion is
// exact: bf16's 8-bit significand fits fp16's 11 bits wherever x s is in
// fp16's normal range, and only values more than 2^28 below the row's largest
// lose bits (below 2^-38 of it they become zero). inf and NaN stay inf and
// NaN. The wide kernel multiplies its fp32 sums by inv[m] (exact) and rounds
// once to bf16.
template <bool PERMUTE>
__global__ __launch_bounds__(kThreads) void scale_rows_kernel(const uint16_t *__restrict__ x, _Float16 *__restrict__ xp,
                                                             float *__restrict__ inv, int64_t K) {
    __shared__ float wave_max[kThreads / 64];
    const int64_t m = blockIdx.x;
    const uint16_t *row = x + m * K;
    _Float16 *out = xp + m * K;
    // K is a multiple of 128, so rows of x and xp start 16-byte aligned
    // whenever x and xp do: then 16-byte reads (8 values) and writes, else
    // one value at a time.
    const bool wide = ((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(xp)) & 15u) == 0;
    auto finite_abs = [](uint32_t bits) {
        const float v = __uint_as_float(bits);
        return __builtin_isfinite(v) ? fabsf(v) : 0.0f;
    };
    float big = 0.0f;
    if (wide) {
        const uint4 *r4 = reinterpret_cast<const uint4 *>(row);
        for (int64_t c = threadIdx.x; c < K / 8; c += kThreads) {
            const uint4 v = r4[c];
            const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
            for (int i = 0; i < 4; ++i)
                big = fmaxf(big, fmaxf(finite_abs(w[i] << 16), finite_abs(w[i] & 0xffff0000u)));
        }
    } else {
        for (int64_t k = threadIdx.x; k < K; k += kThreads)
            big = fmaxf(big, finite_abs(static_cast<uint32_t>(row[k]) << 16));
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) big = fmaxf(big, __shfl_xor(big, off, 64));
    if ((threadIdx.x & 63) == 0) wave_max[threadIdx.x >> 6] = big;
    __syncthreads();
    big = wave_max[0];
#pragma unroll
    for (int w = 1; w < kThreads / 64; ++w) big = fmaxf(big, wave_max[w]);
    int e = 0;
    if (big > 0.0f) {
        int exponent;
        frexpf(big, &exponent);  // big = f 2^exponent, f in [0.5, 1)
        e = min(14 - (exponent - 1), 126);
    }
    const float s = ldexpf(1.0f, e);
    if (threadIdx.x == 0) inv[m] = ldexpf(1.0f, -e);
    // 4-half units: unit u of the copy is unit direct_source_unit(u) of x
    // (PERMUTE) or unit u.
    auto scaled = [&](uint32_t bits) { return static_cast<_Float16>(__uint_as_float(bits) * s); };
    auto pair = [&](uint32_t w) {  // two bf16 values -> two fp16 values, low first
        const _Float16 h[2] = {scaled(w << 16), scaled(w & 0xffff0000u)};
        return __builtin_bit_cast(uint32_t, h);
    };
    if (wide) {
        const uint2 *r2 = reinterpret_cast<const uint2 *>(row);
        uint4 *o4 = reinterpret_cast<uint4 *>(out);
        for (int64_t c = threadIdx.x; c < K / 8; c += kThreads) {  // copy chunk c: units 2c, 2c + 1
            const int64_t group = c >> 4;
            const int u = static_cast<int>(c & 15) * 2;
            const uint2 a = r2[group * 32 + (PERMUTE ? direct_source_unit(u) : u)];
            const uint2 b = r2[group * 32 + (PERMUTE ? direct_source_unit(u + 1) : u + 1)];
            o4[c] = uint4{pair(a.x), pair(a.y), pair(b.x), pair(b.y)};
        }
    } else {
        for (int64_t unit = threadIdx.x; unit < K / 4; unit += kThreads) {
            const int64_t group = unit >> 5;
            const int u = static_cast<int>(unit & 31);
            const int64_t src = group * 32 + (PERMUTE ? direct_source_unit(u) : u);
            _Float16 h[4];
#pragma unroll
            for (int j = 0; j < 4; ++j) h[j] = scaled(static_cast<uint32_t>(row[src * 4 + j]) << 16);
            *reinterpret_cast<uint2 *>(out + unit * 4) = __builtin_bit_cast(uint2, h);
        }
    }
}

// Uses every decoded dword in an empty asm statement, so the decode of a
// group stays in the step that computes it (else it is sunk past the step's
// barrier toward the next step's MFMAs).
__device__ __forceinline__ void pin_decoded(const uint32_t (&a)[32]) {
#pragma unroll
    for (int q = 0; q < 32; ++q) asm volatile("" ::"v"(a[q]));
}

typedef __attribute__((address_space(3))) void lds_void;

// 16-byte-per-lane LDS-DMA through a buffer resource (gfx950). A plain
// function, so that its arguments are checked once and not per template
// instance: the host pass of a kernel template fails to instantiate a direct
// call whose arguments depend on the template parameter.
__device__ __forceinline__ void buffer_dma16(__amdgpu_buffer_rsrc_t rsrc, void *lds, uint32_t voffset,
                                             uint32_t soffset) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, (lds_void *)lds, 16, voffset, soffset, 0, 0);
}
// The same with 4 bytes per lane (one 256-byte row of a group per instruction).
__device__ __forceinline__ void buffer_dma4(__amdgpu_buffer_rsrc_t rsrc, void *lds, uint32_t voffset,
                                            uint32_t soffset) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, (lds_void *)lds, 4, voffset, soffset, 0, 0);
}

// BF: the activations were bf16 (scale_rows_kernel): each output value is
// the fp32 sum times its activation row's inv, rounded once to bf16.
template <int NB, bool BF>
__global__ __launch_bounds__(kWideThreads) void wide_gemm_kernel(
    const uint32_t *__restrict__ packed, const _Float16 *__restrict__ xp, uint16_t *__restrict__ y,
    float *__restrict__ partial, unsigned *__restrict__ counters, const float *__restrict__ row_inv,
    WideGeometry geo) {
    constexpr int kCols = NB * 32;                  // activation rows per tile
    constexpr int kXBytes = wide_x_bytes(NB);
    constexpr int kRing = wide_ring(NB);
    constexpr int kFragFloats = wide_frag_floats(NB);
    // LDS: a ring of activation buffers, then a ring of word buffers. Activation
    // rows are 256 bytes; 16-byte chunk c of row r is stored at chunk
    // c ^ (r & 15), so the sixteen rows one cycle of a 16-byte-per-lane read
    // serves (64 banks) hit distinct banks. Word buffer: word j of row r of
    // 64-row block b at byte b * 1792 + j * 256 + r * 4 (the packed layout).
    extern __shared__ __attribute__((aligned(16))) unsigned char wide_lds[];
    __shared__ unsigned s_last;
    __shared__ unsigned s_published;
    __shared__ uint32_t selectors[tq1_bytes::kSelEntries];

    const int tid = threadIdx.x;
    if (tid < tq1_bytes::kSelEntries) selectors[tid] = tq1_bytes::selector_entry(tid);  // read after the first barrier
    const char *const sel_bytes = reinterpret_cast<const char *>(selectors);
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // uniform: LDS-DMA bases go in M0
    const bool upper = lane >= 32;
    const int P = gridDim.x;
    // Workgroups go to the 8 XCDs round-robin by launch index; with this
    // order each XCD runs one contiguous eighth of the unit sequence, so its
    // L2 serves the activation blocks of its own tiles only and most tiles'
    // contributors share an XCD. The results do not depend on the placement.
    const int p = P % kXcds == 0 ? (blockIdx.x % kXcds) * (P / kXcds) + blockIdx.x / kXcds : blockIdx.x;
    const int G = geo.G;
    const int row_bytes = G * kBlockWeights * 2;  // one activation row
    const int u_begin = wide_unit_begin(geo.units, p, P);
    const int u_end = wide_unit_begin(geo.units, p + 1, P);
    // Phase stamps of the profile build: 0 start, 1 the first unit's operands
    // in LDS, 5 a segment summed, 6 its arrival counted; for a tile this
    // workgroup reduces, 7 the others' partials published and 8 the tile
    // stored (the last segment's stamps are the ones kept).
    const int wide_wave_id = p * kWideWaves + wave;
    (void)wide_wave_id;
    TQ1_PHASE(wide_wave_id, 0);
    TQ1_PHASE_XCC(wide_wave_id);

    if (u_begin >= u_end) return;
    const int last_u = u_end - 1;

    auto tile_of = [&](int u) { return u / G; };
    // Position of a unit: weight row tile tn, activation tile tm, group g
    // (advanced by one unit at a time, so no division runs in the loop).
    struct Cursor {
        int tn, tm, g;
    };
    auto cursor_of = [&](int u) {
        const int t = tile_of(u);
        return Cursor{t % geo.tiles_n, t / geo.tiles_n, u - t * G};
    };
    auto advance = [&](Cursor &c, int by) {  // by is 0 or 1; selects, no branches
        const int g1 = c.g + by;
        const int wrap = g1 == G;
        c.g = wrap ? 0 : g1;
        const int tn1 = c.tn + wrap;
        const int wrap2 = tn1 == geo.tiles_n;
        c.tn = wrap2 ? 0 : tn1;
        c.tm += wrap2;
    };

    unsigned char *const xbuf0 = wide_lds;
    unsigned char *const wbuf0 = wide_lds + kRing * kXBytes;
    // DMA of a group's activation tile, row r of it at byte 256 r with its
    // 16-byte chunks XOR-swizzled by r mod 16 (logical chunk c at c ^ (r % 16)).
    // Four or eight blocks read the permuted copy xp (the direct K order) by
    // 16-byte DMA: 8 NB blocks of 1 KiB (4 rows), NB per wave; lane l of
    // block b fills row 4b + l/16, stored chunk l%16. Block b = NB w + j starts
    // at row 4b: the lane part of the offset depends on b % 4 only (row % 16),
    // the rest (16 (b / 4) rows) is uniform. One or two blocks read x itself by
    // 4-byte DMA, one row per instruction, each lane fetching the dword its
    // swizzled position holds in the K order -- no pre-pass, whose launch
    // would cost more than these few rows.
    constexpr bool kDirectX = NB <= 2;
    constexpr int kRowsPerWave = kCols / kWideWaves;  // 4 or 8 when kDirectX
    constexpr int kVoff = kDirectX ? kRowsPerWave : (NB % 4 == 0 ? 4 : NB);
    constexpr int kXDmaPerWave = kDirectX ? kRowsPerWave : NB;
    uint32_t voff_x[kVoff];
#pragma unroll
    for (int j = 0; j < kVoff; ++j) {
        if (kDirectX) {
            const int row = wave * kRowsPerWave + j;
            const int chunk = (lane >> 2) ^ (row & 15);  // logical chunk at position lane / 4
            const int unit = direct_source_unit(2 * chunk + ((lane >> 1) & 1));
            voff_x[j] = static_cast<uint32_t>(unit * 8 + (lane & 1) * 4);
        } else {
            const int row = 4 * ((wave * NB + j) & 3) + (lane >> 4);
            voff_x[j] = static_cast<uint32_t>(row * row_bytes + (((lane & 15) ^ (row & 15)) * 16));
        }
    }
    auto issue_x = [&](const Cursor &c, int buf) {
        const int m0 = c.tm * kCols;
        const __amdgpu_buffer_rsrc_t rx = __builtin_amdgcn_make_buffer_rsrc(
            const_cast<_Float16 *>(xp) + static_cast<int64_t>(m0) * (row_bytes / 2), 0,
            min(kCols, geo.M - m0) * row_bytes, kBufferRsrcFlags);
        if constexpr (kDirectX) {
#pragma unroll
            for (int j = 0; j < kRowsPerWave; ++j) {
                const int r = wave * kRowsPerWave + j;
                buffer_dma4(rx, xbuf0 + buf * kXBytes + r * 256, voff_x[j], r * row_bytes + c.g * 256);
            }
        } else {
#pragma unroll
            for (int j = 0; j < NB; ++j) {
                const int b = wave * NB + j;
                buffer_dma16(rx, xbuf0 + buf * kXBytes + b * 1024, voff_x[j % kVoff],
                             (b >> 2) * 16 * row_bytes + c.g * 256);
            }
        }
    };
    // DMA of a group's words: 64-row block b = wave / 2, words 0-3 by the even
    // wave and 4-6 by the odd one (its fourth load repeats word 6).
    const int rb = wave >> 1;
    const uint32_t voff_w = static_cast<uint32_t>(rb * G * kTileGroupWords * 4 + lane * 4);
    auto issue_w = [&](const Cursor &c, int buf) {
        const int rb0 = c.tn * kWideRowBlocks;
        const __amdgpu_buffer_rsrc_t rw = __builtin_amdgcn_make_buffer_rsrc(
            const_cast<uint32_t *>(packed) + static_cast<int64_t>(rb0) * G * kTileGroupWords, 0,
            min(kWideRowBlocks, geo.row_blocks - rb0) * G * kTileGroupWords * 4, kBufferRsrcFlags);
#pragma unroll
        for (int jj = 0; jj < 4; ++jj) {
            const int j = min((wave & 1) * 4 + jj, kBlockWords - 1);
            __builtin_amdgcn_raw_ptr_buffer_load_lds(
                rw, (lds_void *)(wbuf0 + buf * kWideWBytes + rb * (kTileGroupWords * 4) + j * 256), 4, voff_w,
                c.g * (kTileGroupWords * 4) + j * 256, 0, 0);
        }
    };
    // The five words lane l decodes: words 3h .. 3h+3 (h = l / 32) and the
    // other end word (6 for h = 0, 0 -- the scale -- for h = 1).
    const int wrow = rb * (kTileGroupWords * 4) + ((wave & 1) * 32 + (lane & 31)) * 4;
    auto read_words = [&](uint32_t (&w)[5], int buf) {
        const uint32_t *base = reinterpret_cast<const uint32_t *>(wbuf0 + buf * kWideWBytes + wrow);
        const int first = upper ? 3 : 0;
#pragma unroll
        for (int j = 0; j < 4; ++j) w[j] = base[(first + j) * kTileRows];
        w[4] = base[(upper ? 0 : 6) * kTileRows];
    };

    // B fragment of MFMA step st, activation block nb: row 32 nb + (lane & 31),
    // logical positions 64h + 8st .. +8, i.e. chunk 8h + st of the row, stored
    // at chunk (8h ^ (lane & 8)) | (st ^ (lane & 7)).
    const int frag_row = (lane & 31) * kBlockWeights + (((upper ? 8 : 0) ^ (lane & 8)) * 8);
    const int frag_l7 = lane & 7;

    float16v acc[NB];
    auto zero_acc = [&]() {
#pragma unroll
        for (int nb = 0; nb < NB; ++nb)
#pragma unroll
            for (int e = 0; e < 16; ++e) acc[nb][e] = 0.0f;
    };
    zero_acc();

    // One group step on a single register buffer `a` (32 dwords): stage st
    // runs MFMA step st of the current group from dwords 4st..4st+3
    // (activation buffer buf). The decode of the next group's words w
    // overwrites dwords 4(st-1)..4(st-1)+3 at stage st (the last stage its
    // own as well), a stage after the MFMAs that read them, and the selector
    // table reads of each window run a stage or more ahead of the perms that
    // take them: no stage waits on the LDS between its MFMAs.
    auto step = [&](uint32_t (&a)[32], const uint32_t (&w)[5], int buf, bool mfma) {
        uint32_t th = 0, tl = 0;
        uint32_t sel[32], late[7];
        const uint32_t u[4] = {w[0], w[1], w[2], w[3]};
        WindowSplits sp;
        const _Float16 *xb = reinterpret_cast<const _Float16 *>(xbuf0 + buf * kXBytes);
        auto frag = [&](int st, int nb) {
            return *reinterpret_cast<const half8 *>(xb + nb * 32 * kBlockWeights + frag_row + ((st ^ frag_l7) * 8));
        };
        // Eight blocks: activation fragments in two sets of four, a set read
        // for stage st + 1 as soon as the MFMAs of stage st have consumed it,
        // so the reads overlap the other set's MFMAs. Fewer blocks: a stage's
        // fragments are read at its start.
        half8 bx[4], by[4];
        if (NB == 8 && mfma) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                bx[i] = frag(0, i);
                by[i] = frag(0, 4 + i);
            }
        }
#pragma unroll
        for (int st = 0; st < 8; ++st) {
            // Stages are scheduling regions: the decode of a stage is not
            // hoisted into earlier ones (its selectors would all be live at
            // once).
            __builtin_amdgcn_sched_barrier(0);
            if (NB < 8 && mfma) {
                half8 af;
                {
                    uint4 v = {a[4 * st], a[4 * st + 1], a[4 * st + 2], a[4 * st + 3]};
                    af = *reinterpret_cast<half8 *>(&v);
                }
                half8 bf[NB];
#pragma unroll
                for (int nb = 0; nb < NB; ++nb) bf[nb] = frag(st, nb);
#pragma unroll
                for (int nb = 0; nb < NB; ++nb)
                    acc[nb] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af, bf[nb], acc[nb], 0, 0, 0);
                // the fragment reads first, then each MFMA with a share of the decode
                __builtin_amdgcn_sched_group_barrier(0x100, NB, 0);
#pragma unroll
                for (int nb = 0; nb < NB; ++nb) {
                    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                    __builtin_amdgcn_sched_group_barrier(0x002, 24 / NB, 0);
                }
            }
            if (NB == 8 && mfma) {
                half8 af;
                {
                    uint4 v = {a[4 * st], a[4 * st + 1], a[4 * st + 2], a[4 * st + 3]};
                    af = *reinterpret_cast<half8 *>(&v);
                }
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    acc[i % NB] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af, bx[i], acc[i % NB], 0, 0, 0);
                if (st < 7) {
#pragma unroll
                    for (int i = 0; i < 4; ++i) bx[i] = frag(st + 1, i);
                }
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    acc[(4 + i) % NB] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af, by[i], acc[(4 + i) % NB], 0, 0, 0);
                if (st < 7) {
#pragma unroll
                    for (int i = 0; i < 4; ++i) by[i] = frag(st + 1, 4 + i);
                }
                // each MFMA followed by a share of the decode, the next
                // stage's reads after the MFMAs of their set
#pragma unroll
                for (int half = 0; half < 2; ++half) {
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                        __builtin_amdgcn_sched_group_barrier(0x002, 3, 0);
                    }
                    if (st < 7) __builtin_amdgcn_sched_group_barrier(0x100, 4, 0);
                }
            }
            // selectors of windows 0-1 at stage 0, 2 at 1, 3 at 2, 4 at 3, 5 at
            // 4 and the tail's at 5; stage st's perms take selectors
            // 4(st-1) .. 4(st-1)+3, which come from windows read by stage st-1
            if (st == 0) {
                scale_tables((upper ? w[4] : w[0]) & 0xffffu, th, tl);
                sp = window_splits(u, 0);
                window_selectors(sp, 0, 0, sel_bytes, sel, late);
                window_selectors(sp, 0, 1, sel_bytes, sel, late);
            } else if (st == 1 || st == 3) {
                sp = window_splits(u, (st + 1) / 2);
                window_selectors(sp, (st + 1) / 2, 0, sel_bytes, sel, late);
            } else if (st == 2 || st == 4) {
                window_selectors(sp, st / 2, 1, sel_bytes, sel, late);
            } else if (st == 5) {
                tail_selectors(upper ? w[3] : w[4], upper, sel_bytes, sel, late);
            }
            if (st > 0) {
#pragma unroll
                for (int q = 4 * (st - 1); q < 4 * st; ++q)
                    a[q] = __builtin_amdgcn_perm(th, tl, full_selector(sel, late, q));
            }
            if (st == 7) {
#pragma unroll
                for (int q = 28; q < 32; ++q) a[q] = __builtin_amdgcn_perm(th, tl, full_selector(sel, late, q));
            }
        }
    };

    // Writes the 16 values of fragment nb of tile t. D[i][j] of a 32x32 tile
    // sits in lane j + 32 * ((i / 4) % 2), item 4 * (i / 8) + i % 4; i is a
    // weight row (32 wave + i), j an activation row (32 nb + j). Lanes j and
    // j + 32 swap half their values (as fp16 pairs) so that each holds two
    // runs of 8 consecutive rows: two 16-byte stores per lane, not 16 scattered
    // 2-byte ones. Every lane takes part in the swap; stores are guarded.
    auto out_bits = [&](float v) -> uint32_t {
        if constexpr (BF)
            return from_f32<bf16_t>(v).bits;
        else
            return __builtin_bit_cast(uint16_t, static_cast<_Float16>(v));
    };
    auto store_frag = [&](int t, int nb, const float *vals) {
        const int m = (t / geo.tiles_n) * kCols + nb * 32 + (lane & 31);
        float sc = 1.0f;
        if constexpr (BF) sc = row_inv[min(m, geo.M - 1)];
        uint32_t h[4][2];
#pragma unroll
        for (int qq = 0; qq < 4; ++qq)
#pragma unroll
            for (int k = 0; k < 2; ++k)
                h[qq][k] = out_bits(vals[4 * qq + 2 * k] * sc) | (out_bits(vals[4 * qq + 2 * k + 1] * sc) << 16);
        // rows 8qq + 4(lane / 32) + e; the lower lane keeps runs qq = 0, 2, the upper qq = 1, 3
        uint32_t r[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const uint32_t send = upper ? h[(k >> 1) * 2][k & 1] : h[(k >> 1) * 2 + 1][k & 1];
            r[k] = static_cast<uint32_t>(__builtin_amdgcn_ds_bpermute((lane ^ 32) << 2, static_cast<int>(send)));
        }
        if (m >= geo.M) return;
        uint16_t *yrow = y + static_cast<int64_t>(m) * geo.N;
#pragma unroll
        for (int run = 0; run < 2; ++run) {  // rows 16 run + 8 (lane / 32) .. + 8
            const int n = (t % geo.tiles_n) * kWideRows + wave * 32 + 16 * run + (upper ? 8 : 0);
            const uint32_t *own = h[2 * run + (upper ? 1 : 0)];
            uint4 v;
            if (upper) v = uint4{r[2 * run], r[2 * run + 1], own[0], own[1]};
            else v = uint4{own[0], own[1], r[2 * run], r[2 * run + 1]};
            if (geo.vector_rows && n + 8 <= geo.N) {
                *reinterpret_cast<uint4 *>(yrow + n) = v;
            } else {
                const uint32_t d[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
                for (int e = 0; e < 8; ++e)
                    if (n + e < geo.N) yrow[n + e] = static_cast<uint16_t>(d[e >> 1] >> (16 * (e & 1)));
            }
        }
    };
    // Tile t as NaN (fp16 0x7e00, bf16 0x7fc0), the rows store_frag writes.
    auto store_nan_tile = [&](int t) {
        const uint16_t nan16 = BF ? 0x7fc0 : 0x7e00;
#pragma unroll 1
        for (int nb = 0; nb < NB; ++nb) {
            const int m = (t / geo.tiles_n) * kCols + nb * 32 + (lane & 31);
            if (m >= geo.M) continue;
            uint16_t *yrow = y + static_cast<int64_t>(m) * geo.N;
#pragma unroll 1
            for (int run = 0; run < 2; ++run) {
                const int n = (t % geo.tiles_n) * kWideRows + wave * 32 + 16 * run + (upper ? 8 : 0);
                for (int e = 0; e < 8; ++e)
                    if (n + e < geo.N) yrow[n + e] = nan16;
            }
        }
    };
    // Stream-K reduction. A tile split over workgroups q0..q1 is summed in
    // workgroup order by the last of them to arrive (counters[t] counts
    // arrivals), from its own accumulators and the partials the others stored
    // (counters[kWideTileSlots + t] counts those published). A workgroup that
    // is not last stores its partial and publishes it only after the next
    // step's vmcnt(0) and barrier, so no step waits for the stores; the last
    // arriver waits for the publications, which never wait on anything.
    int pending = -1;  // tile of a stored, not yet published partial (uniform)
    auto publish = [&]() {  // after a vmcnt(0) and a barrier: the stores are complete
        if (pending >= 0 && tid == 0)
            __hip_atomic_fetch_add(counters + kWideTileSlots + pending, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        pending = -1;
    };
    // Partials: per workgroup two slots (0 = its first segment, 1 = its last),
    // per wave NB fragments x 4 runs of (64 lanes x 4 floats), device-coherent
    // 16-byte accesses (sc1).
    const __amdgpu_buffer_rsrc_t rp =
        __builtin_amdgcn_make_buffer_rsrc(partial, 0, P * 2 * kWideWaves * kFragFloats * 4, kBufferRsrcFlags);
    const uint32_t voff_p = static_cast<uint32_t>((wave * kFragFloats + lane * 4) * 4);
    constexpr int kDeviceCoherent = 16;  // cache policy SC1
    auto slot_base = [&](int q, int slot) { return (q * 2 + slot) * kWideWaves * kFragFloats * 4; };
    // Emits tile t, whose segment here is [seg_begin, seg_end): directly if it
    // is the whole tile, else through the reduction above.
    auto emit = [&](int t, int seg_begin, int seg_end) {
        const int tu0 = t * G, tu1 = tu0 + G;
        if (seg_begin == tu0 && seg_end == tu1) {
#pragma unroll
            for (int nb = 0; nb < NB; ++nb) {
                float v[16];
#pragma unroll
                for (int e = 0; e < 16; ++e) v[e] = acc[nb][e];
                store_frag(t, nb, v);
            }
            return;
        }
        const int q0 = wide_owner(geo.units, tu0, P), q1 = wide_owner(geo.units, tu1 - 1, P);
        // With the workspace's error word set (read beside the arrival, in
        // flight at the same time), an earlier reduction gave up and the
        // counters may be stale: every contributor writes the tile as NaN,
        // until the host zeroes the workspace.
        if (tid == 0) {
            const unsigned word =
                __hip_atomic_load(counters + kWorkspaceErrorSlot, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            const unsigned old = __hip_atomic_fetch_add(counters + t, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            s_last = word ? 2u : (old == static_cast<unsigned>(q1 - q0) ? 1u : 0u);
        }
        __syncthreads();
        TQ1_PHASE(wide_wave_id, 6);
        if (s_last == 2u) {
            store_nan_tile(t);
            return;
        }
        if (!s_last) {
            const int base = slot_base(p, seg_begin == u_begin ? 0 : 1);
#pragma unroll
            for (int nb = 0; nb < NB; ++nb)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const f32x4 v = {acc[nb][4 * r], acc[nb][4 * r + 1], acc[nb][4 * r + 2], acc[nb][4 * r + 3]};
                    __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, v), rp, voff_p,
                                                           base + (nb * 4 + r) * 1024, kDeviceCoherent);
                }
            pending = t;
            return;
        }
        // Last to arrive: wait (bounded) until the others' partials are published.
        // A wait that gives up writes the tile as NaN (it sums nothing), sets
        // the workspace error word and leaves both counters as they are: a
        // late publication cannot carry into the next call, which finds the
        // word set and refuses; the host zeroes the workspace after reading it.
        if (tid == 0) {
            bool published = false;
            for (int spin = 0; spin <= geo.spin_limit; ++spin) {
                if (__hip_atomic_load(counters + kWideTileSlots + t, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) >=
                    static_cast<unsigned>(q1 - q0)) {
                    published = true;
                    break;
                }
                __builtin_amdgcn_s_sleep(2);
            }
            s_published = published;
            if (!published)
                __hip_atomic_fetch_or(counters + kWorkspaceErrorSlot, 2u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        __syncthreads();
        TQ1_PHASE(wide_wave_id, 7);
        if (!s_published) {
            store_nan_tile(t);
            return;
        }
        // The sum runs in workgroup order q0..q1: the partials of q0..p-1, this
        // workgroup's accumulators, then the partials of p+1..q1. It is formed
        // in place in acc -- (prefix) + acc equals acc + (prefix) exactly in
        // fp32 -- in batches of kRB fragments whose loads are all in flight at
        // once: the reduction at the end of a launch costs one memory round
        // trip per batch and contributor, not one per fragment (batches of two
        // for eight-block tiles, whose accumulators leave no more registers).
        constexpr int kRB = NB == 8 ? 2 : (NB < 4 ? NB : 4);
        auto load_batch = [&](float (&v)[kRB][16], int q, int nb0) {
            // The tile is contributor q's first segment unless q starts before it.
            const int base = slot_base(q, wide_unit_begin(geo.units, q, P) >= tu0 ? 0 : 1);
#pragma unroll
            for (int i = 0; i < kRB; ++i)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const f32x4 f = __builtin_bit_cast(
                        f32x4, __builtin_amdgcn_raw_buffer_load_b128(rp, voff_p, base + ((nb0 + i) * 4 + r) * 1024,
                                                                      kDeviceCoherent));
                    v[i][4 * r] = f.x;
                    v[i][4 * r + 1] = f.y;
                    v[i][4 * r + 2] = f.z;
                    v[i][4 * r + 3] = f.w;
                }
        };
#pragma unroll
        for (int nb0 = 0; nb0 < NB; nb0 += kRB) {
            float v[kRB][16];
            if (p > q0) {
                load_batch(v, q0, nb0);
                for (int q = q0 + 1; q < p; ++q) {
                    float w2[kRB][16];
                    load_batch(w2, q, nb0);
#pragma unroll
                    for (int i = 0; i < kRB; ++i)
#pragma unroll
                        for (int e = 0; e < 16; ++e) v[i][e] += w2[i][e];
                }
#pragma unroll
                for (int i = 0; i < kRB; ++i)
#pragma unroll
                    for (int e = 0; e < 16; ++e) acc[nb0 + i][e] = v[i][e] + acc[nb0 + i][e];
            }
            for (int q = p + 1; q <= q1; ++q) {
                load_batch(v, q, nb0);
#pragma unroll
                for (int i = 0; i < kRB; ++i)
#pragma unroll
                    for (int e = 0; e < 16; ++e) acc[nb0 + i][e] += v[i][e];
            }
#pragma unroll
            for (int i = 0; i < kRB; ++i) {
                float out[16];
#pragma unroll
                for (int e = 0; e < 16; ++e) out[e] = acc[nb0 + i][e];
                store_frag(t, nb0 + i, out);
            }
        }
        if (tid == 0) {
            __hip_atomic_store(counters + t, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_store(counters + kWideTileSlots + t, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        TQ1_PHASE(wide_wave_id, 8);
    };

    // Prefetch cursors: activations kRing - 1 units ahead, words kRing; no
    // DMA is issued past the last unit (uniform branches). Ring slot of unit
    // v: v % kRing.
    int cx_u = u_begin, cw_u = u_begin;
    Cursor cx = cursor_of(cx_u), cw = cursor_of(cw_u);
    auto next_x = [&]() {
        ++cx_u;
        advance(cx, 1);
    };
    auto next_w = [&]() {
        ++cw_u;
        advance(cw, 1);
    };
    uint32_t a[32];
    {
        for (int v = 0; v < kRing - 1; ++v) {
            if (cx_u <= last_u) issue_x(cx, (u_begin + v) & (kRing - 1));
            next_x();
        }
        for (int v = 0; v < kRing; ++v) {
            if (cw_u <= last_u) issue_w(cw, (u_begin + v) & (kRing - 1));
            next_w();
        }
        wait_vector_memory();
        __syncthreads();
        TQ1_PHASE(wide_wave_id, 1);
        uint32_t w[5];
        read_words(w, u_begin & (kRing - 1));
        step(a, w, u_begin & (kRing - 1), false);  // decode only (0 * inf activations would be NaN)
        pin_decoded(a);
        __syncthreads();  // every wave has read the words the first step overwrites
    }

    // s_waitcnt vmcnt(n): at the end of step u the activations of u+1 and the
    // words of u+2 -- issued kRing - 2 steps earlier, or before the loop --
    // must have landed; the DMAs of the kRing - 2 later steps may stay in
    // flight (gfx9 encoding: vmcnt bits 3:0 and 15:14, other counters idle).
    constexpr int kInFlight = (kRing - 2) * (kXDmaPerWave + 4);
    constexpr unsigned kWaitRing = (kInFlight & 15) | ((kInFlight >> 4) << 14) | 0x0f70;
    static_assert(kInFlight <= 63, "vmcnt holds at most 63");
    // Segments: maximal runs of this workgroup's units within one tile; the
    // pipeline runs on across them (the decode and prefetches of a segment's
    // last step already belong to the next one).
    for (int u = u_begin; u < u_end;) {
        const int t = tile_of(u);
        const int seg_begin = u;
        const int seg_end = min(u_end, (t + 1) * G);
        zero_acc();
        for (; u < seg_end; ++u) {
            const int slot = u & (kRing - 1);
            __builtin_amdgcn_sched_barrier(0);
            asm volatile("" ::: "memory");
            if (cx_u <= last_u) issue_x(cx, (slot + kRing - 1) & (kRing - 1));
            if (cw_u <= last_u) issue_w(cw, slot);
            asm volatile("" ::: "memory");
            __builtin_amdgcn_sched_barrier(0);
            next_x();
            next_w();
            uint32_t w[5];
            read_words(w, (slot + 1) & (kRing - 1));
            step(a, w, slot, true);
            pin_decoded(a);
            __builtin_amdgcn_sched_barrier(0);
            // A partial stored after the previous step is published once
            // every store of this workgroup is complete; near the end of the
            // range fewer DMAs are in flight than the counted wait assumes.
            if (kRing == 2 || pending >= 0 || u + kRing - 1 > last_u) wait_vector_memory();
            else __builtin_amdgcn_s_waitcnt(kWaitRing);
            asm volatile("s_barrier" ::: "memory");
            publish();
        }
        TQ1_PHASE(wide_wave_id, 5);
        emit(t, seg_begin, seg_end);
    }
    wait_vector_memory();
    __syncthreads();
    publish();
}


// ---------------------------------------------------------------------------
// Host-side geometry
// ---------------------------------------------------------------------------
int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }

int64_t packed_words(int64_t rows, int64_t columns) {
    return ceil_div(rows, kTileRows) * (columns / kBlockWeights) * kTileGroupWords;
}

// Dynamic LDS above 64 KiB needs hipFuncSetAttribute once per kernel and
// device; the set of (kernel, device) pairs already opted in is shared by all
// threads.
int ensure_lds_attribute(const void *kernel, int bytes) {
    static std::mutex mu;
    static std::set<std::pair<const void *, int>> done;
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return fail(TERNEL_TQ1_EHIP, "hipGetDevice failed");
    std::lock_guard<std::mutex> lock(mu);
    if (done.count({kernel, dev})) return TERNEL_TQ1_OK;
    const hipError_t e = hipFuncSetAttribute(kernel, hipFuncAttributeMaxDynamicSharedMemorySize, bytes);
    if (e != hipSuccess) return fail(TERNEL_TQ1_EHIP, "hipFuncSetAttribute: %s", hipGetErrorString(e));
    done.insert({kernel, dev});
    return TERNEL_TQ1_OK;
}

// Polls of one published value before a kernel's bounded wait gives up and
// sets the workspace error word (a negative limit makes every such wait give
// up at once: the tests' way to drive the error path from the host).
std::atomic<int> g_spin_limit{1 << 22};

int check_dtype(int dtype) {
    if (dtype != TERNEL_TQ1_F16 && dtype != TERNEL_TQ1_BF16 && dtype != TERNEL_TQ1_F32)
        return fail(TERNEL_TQ1_EINVAL, "unsupported dtype code %d", dtype);
    return TERNEL_TQ1_OK;
}

int check_geometry(int64_t M, int64_t rows, int64_t columns) {
    if (rows <= 0 || columns <= 0)
        return fail(TERNEL_TQ1_EINVAL, "tensor dimensions must be positive, got %lldx%lld",
                    static_cast<long long>(rows), static_cast<long long>(columns));
    if (columns % kBlockWeights)
        return fail(TERNEL_TQ1_EINVAL, "%lld columns is not a multiple of the 128-weight group",
                    static_cast<long long>(columns));
    if (M <= 0) return fail(TERNEL_TQ1_EINVAL, "activations have an empty batch dimension");
    if (rows > INT32_MAX - kThreads || M > INT32_MAX || columns / kBlockWeights > INT32_MAX / kTileGroupWords)
        return fail(TERNEL_TQ1_EINVAL, "tensor too large for 32-bit row/batch indices");
    return TERNEL_TQ1_OK;
}

// Above this many K chunks the split-K fix-up costs more than the extra
// workgroups buy (measured, see plan_lut).
constexpr int64_t kLutMaxChunks = 20;
// Split-K partials of one LUT23 launch, at most (a larger batch runs as more
// launches).
constexpr int64_t kLutPartialBytes = int64_t{256} << 20;

// The split-K workspace starts with a fixed region of arrival counters, one per
// (row block, batch tile), that is all-zero between calls. Fixing its size keeps
// that true when one workspace serves calls of different shapes: partials are
// always written past it.
constexpr int kCounterSlots = 16384;
constexpr size_t kCounterRegionBytes = kCounterSlots * sizeof(unsigned);
static_assert(kCounterRegionBytes == kWorkspaceCounterBytes, "one counter region");
// The last counter slot is the workspace's error word: a kernel whose bounded
// wait gave up sets it (ternel_tq1_workspace_error reads it). Counters of every
// kernel stay below it.
constexpr int kErrorSlot = kCounterSlots - 1;
static_assert(kErrorSlot == kWorkspaceErrorSlot, "one error word");
constexpr int kUsableCounters = kCounterSlots - 16;
// Partials of every split kernel start here.
constexpr size_t kPartialOffset = kCounterRegionBytes;

struct LutPlan {
    int batch_tile;
    int waves;         // waves per 64-row tile (compile-time KW)
    int row_tiles;     // 64-row tiles per workgroup (compile-time RT)
    int chunk;         // groups per sub-chunk (compile-time C)
    int chunk_groups;  // groups per workgroup, a multiple of chunk
    int k_split;
    int64_t row_blocks;
    int64_t batch_tiles;        // of one launch
    int64_t launch_vectors;     // activation rows per launch (a batch above it runs in several)
    size_t counter_bytes;
    size_t partial_bytes;
};

bool lut_chunk_supported(int batch_tile, int chunk) {
    if (batch_tile == 4) return chunk == 1 || chunk == 2 || chunk == 4;
    return chunk == 1 || chunk == 2 || chunk == 4 || chunk == 8;
}

int device_cu_count();  // the current device's CUs (256 when it cannot be queried)

// max_partial_bytes bounds one launch's split-K partials (kLutPartialBytes
// unless the workspace is a fixed array).
int plan_lut(int64_t M, int64_t rows, int64_t columns, int batch_tile, int k_split, LutPlan *plan,
             int64_t max_partial_bytes = kLutPartialBytes) {
    const int64_t G = columns / kBlockWeights;
    // Measured on MI355X: one vector per workgroup beats batch tiles of 2 and 4
    // at every 27B shape up to M = 4 (gate/up M=4: 18.3 us vs 20.3 and 25.8);
    // the extra tables and lookups cost more than re-reading the weights from L2.
    if (batch_tile == 0) batch_tile = 1;
    if (batch_tile != 1 && batch_tile != 2 && batch_tile != 4)
        return fail(TERNEL_TQ1_EINVAL, "batch tile must be 1, 2 or 4, got %d", batch_tile);
    plan->batch_tile = batch_tile;
    plan->waves = 1;
    plan->row_tiles = kThreads / kTileRows;
    plan->row_blocks = ceil_div(rows, kThreads);
    plan->batch_tiles = ceil_div(M, batch_tile);
    if (k_split < 0) return fail(TERNEL_TQ1_EINVAL, "k split must be positive, got %d", k_split);
    if (k_split > 0 && G % k_split)
        return fail(TERNEL_TQ1_EINVAL, "k split %d does not divide the tensor's %lld groups per row", k_split,
                    static_cast<long long>(G));
    if (k_split > 0) {
        // A requested split fixes the groups per workgroup; they are walked in
        // sub-chunks of the largest compiled size that divides them, in order,
        // so a split of one keeps the reference's exact summation order.
        plan->chunk_groups = static_cast<int>(G / k_split);
        int c = 1;
        for (int cand : {8, 4, 2, 1})
            if (plan->chunk_groups % cand == 0 && lut_chunk_supported(batch_tile, cand)) {
                c = cand;
                break;
            }
        plan->chunk = c;
        plan->k_split = k_split;
    } else {
        // Measured on MI355X over the 27B shapes (graph-replayed, cold): four
        // groups per workgroup wins (gate/up 10.6 us at k=10 vs 13.1 at k=5 and
        // 13.1 at k=20; QKV, O and the 4096 square likewise), except where that
        // leaves more than kLutMaxChunks K chunks to fix up -- down (G=136) runs
        // 13.3 us at k=17 against 15.3 at k=34 -- where eight groups do.
        int c = 1;
        for (int cand : {4, 2}) {
            if (lut_chunk_supported(batch_tile, cand) && G % cand == 0) {
                c = cand;
                break;
            }
        }
        if (G / c > kLutMaxChunks && G % 8 == 0 && lut_chunk_supported(batch_tile, 8)) c = 8;
        plan->chunk = c;
        plan->chunk_groups = c;
        plan->k_split = static_cast<int>(G / c);
    }
    // Two waves per row tile, each summing half of a sub-chunk's blocks, for
    // one vector per workgroup: a wave's blocks are all in flight before its
    // first sum. That pays while the grid is resident at once (three 512-thread
    // workgroups per CU) or a chunk has eight blocks; a longer grid streams
    // better with single-wave tiles. Measured on MI355X (graph-replayed, cold,
    // us, one wave -> two): M=1 down 12.4 -> 11.0, QKV 8.4 -> 8.0, gate/up
    // 9.9 -> 9.8; M=2 down 14.7 -> 14.0 but gate/up 13.6 -> 14.3; the 248320-row
    // head 62.6 -> 75.7.
    if (plan->batch_tile == 1 && plan->chunk >= 2 &&
        (plan->chunk >= 8 || plan->row_blocks * plan->batch_tiles * plan->k_split <= 3 * device_cu_count()))
        plan->waves = 2;
    // One vector over a split whose 256-row workgroups number fewer than 1.5
    // per CU (the 340 of down 17408->5120 leave a third of the CUs running two
    // and the rest one): 128-row workgroups, twice as many, even the CUs out.
    // Measured on MI355X (graph-replayed, cold, us, 256 -> 128 rows): down
    // 10.64 -> 10.21, O 8192->5120 8.49 -> 8.27; gate/up (680 workgroups)
    // 9.60 -> 9.74, so not there.
    if (plan->batch_tile == 1 && plan->k_split > 1 &&
        2 * plan->row_blocks * plan->batch_tiles * plan->k_split <= 3 * device_cu_count()) {
        plan->row_tiles = 2;
        plan->row_blocks = ceil_div(rows, plan->row_tiles * kTileRows);
    }
    if (plan->k_split > 65535) return fail(TERNEL_TQ1_EINVAL, "K too large for one launch");
    // A split launch needs one arrival counter per (row block, batch tile):
    // a batch past what the counter region holds runs as several launches
    // (in order on the stream, each leaving its counters zero for the next).
    plan->launch_vectors = M;
    if (plan->k_split > 1 && plan->row_blocks * plan->batch_tiles > kUsableCounters) {
        const int64_t tiles = kUsableCounters / plan->row_blocks;
        if (tiles < 1)
            return fail(TERNEL_TQ1_EINVAL, "%lld row blocks exceed the %d split-K counters",
                        static_cast<long long>(plan->row_blocks), kUsableCounters);
        plan->launch_vectors = tiles * plan->batch_tile;
        plan->batch_tiles = tiles;
    }
    if (plan->batch_tiles > 65535) {
        plan->batch_tiles = 65535;
        plan->launch_vectors = std::min<int64_t>(plan->launch_vectors, 65535 * static_cast<int64_t>(plan->batch_tile));
    }
    if (plan->k_split > 1) {
        // At most max_partial_bytes of partials per launch: fewer vectors per
        // launch, or -- when not even one batch tile fits and the split was
        // automatic -- no split (a grid that tall fills the CUs unsplit).
        const int64_t per_vector = static_cast<int64_t>(plan->k_split) * rows * sizeof(float);
        int64_t fit = max_partial_bytes / per_vector;
        fit -= fit % plan->batch_tile;
        if (fit < plan->batch_tile && k_split == 0) {
            plan->k_split = 1;
            plan->chunk_groups = static_cast<int>(G);
        } else if (fit >= plan->batch_tile && plan->launch_vectors > fit) {
            plan->launch_vectors = fit;
            plan->batch_tiles = fit / plan->batch_tile;
        }
    }
    plan->counter_bytes = plan->k_split > 1 ? kPartialOffset : 0;
    plan->partial_bytes = plan->k_split > 1 ? static_cast<size_t>(plan->k_split) *
                                                  static_cast<size_t>(plan->launch_vectors) * rows * sizeof(float)
                                            : 0;
    return TERNEL_TQ1_OK;
}

template <typename T, int C, int BT, bool GLU = false>
void launch_lut_kernel(const LutPlan &plan, const uint32_t *packed, const void *x, void *y, float *partial,
                       unsigned *counters, int64_t M, int64_t rows, int G, hipStream_t stream) {
    const dim3 grid(static_cast<unsigned>(plan.row_blocks), static_cast<unsigned>(plan.batch_tiles),
                    static_cast<unsigned>(plan.k_split));
#define TQ1_LUT_KERNEL_LAUNCH(KW, RT)                                                                          \
    hipLaunchKernelGGL((lut_gemv_kernel<T, C, BT, GLU, KW, RT>), grid, dim3(KW * RT * kTileRows), 0, stream,     \
                       packed, static_cast<const T *>(x), static_cast<T *>(y), partial, counters,                \
                       static_cast<int>(M), static_cast<int>(rows), G, plan.chunk_groups, plan.k_split)
    if constexpr (BT == 1) {
        if (plan.row_tiles == 2) {
            if constexpr (C >= 2) {
                if (plan.waves == 2) {
                    TQ1_LUT_KERNEL_LAUNCH(2, 2);
                    return;
                }
            }
            TQ1_LUT_KERNEL_LAUNCH(1, 2);
            return;
        }
    }
    if constexpr (BT == 1 && C >= 2) {
        if (plan.waves == 2) {
            TQ1_LUT_KERNEL_LAUNCH(2, 4);
            return;
        }
    }
    TQ1_LUT_KERNEL_LAUNCH(1, 4);
#undef TQ1_LUT_KERNEL_LAUNCH
}

template <typename T>
int launch_lut_once(const uint32_t *packed, const void *x, void *y, int64_t M, int64_t rows, int64_t columns,
                    const LutPlan &plan, void *ws, hipStream_t stream, bool glu);

// Runs the batch as ceil(M / launch_vectors) launches of at most
// launch_vectors activation rows each.
template <typename T>
int launch_lut(const uint32_t *packed, const void *x, void *y, int64_t M, int64_t rows, int64_t columns,
               const LutPlan &plan, void *ws, hipStream_t stream, bool glu = false) {
    const int64_t out_width = glu ? rows / 2 : rows;
    for (int64_t m0 = 0; m0 < M; m0 += plan.launch_vectors) {
        const int64_t mc = std::min(plan.launch_vectors, M - m0);
        LutPlan sub = plan;
        sub.batch_tiles = ceil_div(mc, plan.batch_tile);
        const int rc = launch_lut_once<T>(packed, static_cast<const T *>(x) + m0 * columns,
                                          static_cast<T *>(y) + m0 * out_width, mc, rows, columns, sub, ws, stream, glu);
        if (rc != TERNEL_TQ1_OK) return rc;
    }
    return TERNEL_TQ1_OK;
}

template <typename T>
int launch_lut_once(const uint32_t *packed, const void *x, void *y, int64_t M, int64_t rows, int64_t columns,
                    const LutPlan &plan, void *ws, hipStream_t stream, bool glu) {
    const int G = static_cast<int>(columns / kBlockWeights);
    unsigned *counters = plan.k_split > 1 ? static_cast<unsigned *>(ws) : nullptr;
    float *partial =
        plan.k_split > 1 ? reinterpret_cast<float *>(static_cast<char *>(ws) + plan.counter_bytes) : nullptr;
    if (glu) {  // SwiGLU epilogue: one vector per workgroup
#define TQ1_LUT_GLU_CASE(CC)                                                                          \
        if (plan.chunk == CC && plan.batch_tile == 1) {                                               \
            launch_lut_kernel<T, CC, 1, true>(plan, packed, x, y, partial, counters, M, rows, G, stream); \
            TQ1_LAUNCH_CHECK();                                                                       \
            return TERNEL_TQ1_OK;                                                                     \
        }
        TQ1_LUT_GLU_CASE(1)
        TQ1_LUT_GLU_CASE(2)
        TQ1_LUT_GLU_CASE(4)
        TQ1_LUT_GLU_CASE(8)
#undef TQ1_LUT_GLU_CASE
        return fail(TERNEL_TQ1_EINVAL, "no SwiGLU LUT23 kernel for chunk %d, batch tile %d", plan.chunk,
                    plan.batch_tile);
    }
#define TQ1_LUT_CASE(CC, BB)                                                                         \
    if (plan.chunk == CC && plan.batch_tile == BB) {                                                 \
        launch_lut_kernel<T, CC, BB>(plan, packed, x, y, partial, counters, M, rows, G, stream);     \
        TQ1_LAUNCH_CHECK();                                                                          \
        return TERNEL_TQ1_OK;                                                                        \
    }
    TQ1_LUT_CASE(1, 1)
    TQ1_LUT_CASE(2, 1)
    TQ1_LUT_CASE(4, 1)
    TQ1_LUT_CASE(8, 1)
    TQ1_LUT_CASE(1, 2)
    TQ1_LUT_CASE(2, 2)
    TQ1_LUT_CASE(4, 2)
    TQ1_LUT_CASE(8, 2)
    TQ1_LUT_CASE(1, 4)
    TQ1_LUT_CASE(2, 4)
    TQ1_LUT_CASE(4, 4)
#undef TQ1_LUT_CASE
    return fail(TERNEL_TQ1_EINVAL, "no LUT23 kernel for chunk %d, batch tile %d", plan.chunk, plan.batch_tile);
}

// The M = 1 strip GEMV (strip_gemv_kernel): one workgroup per CU, at most
// one per two rows, for strips of at most 96 rows. Rows of more than 40
// groups (with allow_split) are cut into Z <= 4 K chunks of at most 40 groups,
// one workgroup per (strip, chunk), S = CUs / Z strips, whose row partials
// meet in Z - 1 exchange slots per row in the workspace's counter region
// (strip_workspace_bytes).
constexpr int kStripMaxChunks = 4;
int plan_strip(int64_t rows, int64_t columns, StripGeometry *geo, bool allow_split = true) {
    const int64_t G = columns / kBlockWeights;
    int64_t Z = 1;
    if (G > kStripMaxGroups) {
        Z = ceil_div(G, kStripMaxGroups);
        if (!allow_split || Z > kStripMaxChunks)
            return fail(TERNEL_TQ1_EINVAL, "the strip GEMV takes at most %d groups per row%s",
                        allow_split ? kStripMaxChunks * kStripMaxGroups : kStripMaxGroups,
                        allow_split ? " (in K chunks of at most 40)" : " here");
    }
    const int64_t Gc = ceil_div(G, Z);
    const int64_t units = (rows + 1) / 2;
    const int64_t S = std::max<int64_t>(1, std::min<int64_t>(device_cu_count() / Z, units));
    if (2 * ceil_div(units, S) > kStripMaxRows)
        return fail(TERNEL_TQ1_EINVAL, "strips of %lld rows are past the strip GEMV's %d",
                    static_cast<long long>(2 * ceil_div(units, S)), kStripMaxRows);
    if (S * units > INT32_MAX || rows * G * kBlockWords > INT32_MAX || Z * rows > INT32_MAX)
        return fail(TERNEL_TQ1_EINVAL, "tensor too large for the strip GEMV's 32-bit indices");
    if ((Z - 1) * rows > kUsableCounters)
        return fail(TERNEL_TQ1_EINVAL, "%lld rows in %lld K chunks need more exchange slots than the counter region holds",
                    static_cast<long long>(rows), static_cast<long long>(Z));
    geo->N = static_cast<int>(rows);
    geo->G = static_cast<int>(G);
    geo->S = static_cast<int>(S);
    geo->Z = static_cast<int>(Z);
    geo->Gc = static_cast<int>(Gc);
    geo->P = static_cast<int>(S * Z);
    geo->units = static_cast<int>(units);
    geo->value_base = static_cast<int>((Gc * kLutFloats + 3) / 4 * 4);
    return TERNEL_TQ1_OK;
}

// The split strip GEMV's workspace: the counter region, which holds its
// (Z - 1) N exchange slots (0 without a split).
size_t strip_workspace_bytes(const StripGeometry &geo) { return geo.Z > 1 ? kCounterRegionBytes : 0; }

template <typename T>
int launch_strip(const uint32_t *packed, const void *x, void *y, const StripGeometry &geo, hipStream_t stream,
                 bool glu, void *ws = nullptr) {
    const dim3 grid(static_cast<unsigned>(geo.P));
    const bool stage = sizeof(T) == 2 && (reinterpret_cast<uintptr_t>(x) & 15u) == 0;
    const bool split = geo.Z > 1;
    if (split && (glu || !ws)) return fail(TERNEL_TQ1_EINVAL, "a split strip GEMV needs a workspace and no SwiGLU");
    const T *xt = static_cast<const T *>(x);
    T *yt = static_cast<T *>(y);
    unsigned *slots = split ? static_cast<unsigned *>(ws) : nullptr;
    // Items per wave: the largest strip's ceil(R Gc / 64) items over 16 waves.
    const int64_t max_rows = 2 * ((geo.units + geo.S - 1) / geo.S);
    const int64_t per_wave = ceil_div(ceil_div(max_rows * geo.Gc, 64), kStripWaves);
    if (per_wave > 4) return fail(TERNEL_TQ1_EINVAL, "strip of %lld items per wave", static_cast<long long>(per_wave));
    const bool two_pairs = per_wave > 2;
#define TQ1_STRIP_LAUNCH_P(STAGE, PAIRS)                                                                        \
    do {                                                                                                        \
        if (glu)                                                                                                \
            hipLaunchKernelGGL((strip_gemv_kernel<T, true, STAGE, PAIRS, false>), grid, dim3(kStripThreads), 0,  \
                               stream, packed, xt, yt, slots, geo);                                \
        else if (split)                                                                                         \
            hipLaunchKernelGGL((strip_gemv_kernel<T, false, STAGE, PAIRS, true>), grid, dim3(kStripThreads), 0,  \
                               stream, packed, xt, yt, slots, geo);                                \
        else                                                                                                    \
            hipLaunchKernelGGL((strip_gemv_kernel<T, false, STAGE, PAIRS, false>), grid, dim3(kStripThreads), 0, \
                               stream, packed, xt, yt, slots, geo);                                \
    } while (0)
#define TQ1_STRIP_LAUNCH(STAGE)               \
    do {                                      \
        if (two_pairs)                        \
            TQ1_STRIP_LAUNCH_P(STAGE, 2);     \
        else                                  \
            TQ1_STRIP_LAUNCH_P(STAGE, 1);     \
    } while (0)
    if constexpr (sizeof(T) == 2) {
        if (stage) {
            TQ1_STRIP_LAUNCH(true);
            TQ1_LAUNCH_CHECK();
            return TERNEL_TQ1_OK;
        }
    }
    TQ1_STRIP_LAUNCH(false);
#undef TQ1_STRIP_LAUNCH
#undef TQ1_STRIP_LAUNCH_P
    TQ1_LAUNCH_CHECK();
    return TERNEL_TQ1_OK;
}

// The automatic configuration of one activation vector runs the strip GEMV
// where it applies (the LUT23 kernel above otherwise); allow_split admits
// rows of more than 40 groups (not for the fused SwiGLU form).
bool uses_strip_gemv(int64_t M, int batch_tile, int k_split, int64_t rows, int64_t columns, bool allow_split = true) {
    if (M != 1 || batch_tile != 0 || k_split != 0 || rows < kStripMinRows) return false;
    StripGeometry geo;
    const std::string saved = g_last_error;
    const bool ok = plan_strip(rows, columns, &geo, allow_split) == TERNEL_TQ1_OK;
    snprintf(g_last_error, sizeof(g_last_error), "%s", saved.c_str());
    return ok;
}

struct GemmPlan {
    int k_split;
    int chunk_groups;
    int64_t n_tiles;
    int64_t m_tiles;
};

int largest_divisor_split(int64_t groups_per_row, int64_t workgroups, int64_t target) {
    int64_t budget = target / (workgroups > 0 ? workgroups : 1);
    if (budget < 1) budget = 1;
    if (budget > groups_per_row) budget = groups_per_row;
    for (int64_t k = budget; k > 1; --k)
        if (groups_per_row % k == 0) return static_cast<int>(k);
    return 1;
}

int plan_gemm(int64_t M, int64_t rows, int64_t columns, int k_split, GemmPlan *plan) {
    const int64_t G = columns / kBlockWeights;
    plan->n_tiles = ceil_div(rows, kGemmBN);
    plan->m_tiles = ceil_div(M, kGemmBM);
    if (plan->m_tiles > 65535) return fail(TERNEL_TQ1_EINVAL, "batch too large for one launch");
    if (k_split < 0) return fail(TERNEL_TQ1_EINVAL, "k split must be positive, got %d", k_split);
    if (k_split == 0) {
        const int64_t wgs = plan->n_tiles * plan->m_tiles;
        k_split = wgs >= 512 ? 1 : largest_divisor_split(G, wgs, 512);
    }
    if (G % k_split)
        return fail(TERNEL_TQ1_EINVAL, "k split %d does not divide the tensor's %lld groups per row", k_split,
                    static_cast<long long>(G));
    plan->k_split = k_split;
    plan->chunk_groups = static_cast<int>(G / k_split);
    return TERNEL_TQ1_OK;
}

int launch_gemm(const uint32_t *packed, const void *x, void *y, int64_t M, int64_t rows, int64_t columns,
                const GemmPlan &plan, float *partial, hipStream_t stream) {
    const dim3 grid(static_cast<unsigned>(plan.n_tiles), static_cast<unsigned>(plan.m_tiles),
                    static_cast<unsigned>(plan.k_split));
    hipLaunchKernelGGL(mfma_gemm_kernel, grid, dim3(kThreads), 0, stream, packed,
                       static_cast<const _Float16 *>(x), static_cast<_Float16 *>(y), partial, static_cast<int>(M),
                       static_cast<int>(rows), static_cast<int>(columns / kBlockWeights), plan.chunk_groups);
    TQ1_LAUNCH_CHECK();
    if (partial) {
        const int64_t count = M * rows;
        hipLaunchKernelGGL((reduce_partials_kernel<_Float16>), dim3(static_cast<unsigned>(ceil_div(count, kThreads))),
                           dim3(kThreads), 0, stream, partial, static_cast<_Float16 *>(y), count, plan.k_split);
        TQ1_LAUNCH_CHECK();
    }
    return TERNEL_TQ1_OK;
}

// Direct-fragment form: at most 64 activation rows (two 32-wide MFMA tiles).
constexpr int64_t kDirectMaxBatch = 64;
// Auto split: at least this many workgroups (4 waves each) to fill 256 CUs twice.
constexpr int64_t kDirectTargetWorkgroups = 512;

struct DirectPlan {
    int nb;
    int staged_rows;
    int k_split;
    int chunk_groups;
    int window;  // groups of activations staged in LDS at once
    int64_t row_blocks;
    size_t lds_bytes;
    size_t partial_bytes;
};

int direct_staged_rows(int64_t M) { return M <= 8 ? 8 : (M <= 16 ? 16 : (M <= 32 ? 32 : 64)); }

int plan_direct(int64_t M, int64_t rows, int64_t columns, int k_split, DirectPlan *plan) {
    const int64_t G = columns / kBlockWeights;
    if (M > kDirectMaxBatch)
        return fail(TERNEL_TQ1_EINVAL, "the direct-fragment form takes at most %lld activation rows, got %lld",
                    static_cast<long long>(kDirectMaxBatch), static_cast<long long>(M));
    plan->nb = M > 32 ? 2 : 1;
    plan->staged_rows = direct_staged_rows(M);
    plan->row_blocks = ceil_div(rows, kDirectRows);
    if (k_split < 0) return fail(TERNEL_TQ1_EINVAL, "k split must be positive, got %d", k_split);
    if (k_split == 0) {
        // Measured on MI355X: chunks of a multiple of 8 groups keep the whole
        // K chunk in the 8-step pipeline; take the smallest such split that
        // reaches the workgroup target, else the largest such split. At 32
        // and 64 staged rows chunks of a multiple of 4 qualify too, whose last
        // four groups run the same pipeline (QKV and O at M=32 then run 640
        // workgroups instead of 320: 16.9 and 17.2 us against 18.4 and 18.3,
        // measured with 8-group windows; at M=40-64 QKV 20.7-22.6 us against
        // 23.2-25.2, O 22.8-24.8 against 24.1-26.0); at up to 16 rows 4-group
        // chunks measured slower.
        const int64_t granule = plan->staged_rows >= 32 ? 4 : 8;
        int best = 0;
        for (int64_t k = 1; k <= G; ++k) {
            if (G % k || (G / k) % granule) continue;
            best = static_cast<int>(k);
            if (plan->row_blocks * k >= kDirectTargetWorkgroups) break;
        }
        k_split = best ? best : largest_divisor_split(G, plan->row_blocks, kDirectTargetWorkgroups);
    }
    if (G % k_split)
        return fail(TERNEL_TQ1_EINVAL, "k split %d does not divide the tensor's %lld groups per row", k_split,
                    static_cast<long long>(G));
    if (k_split > 65535) return fail(TERNEL_TQ1_EINVAL, "K too large for one launch");
    if (k_split > 1 && plan->row_blocks > kUsableCounters)
        return fail(TERNEL_TQ1_EINVAL, "%lld row blocks exceed the %d split-K counters",
                    static_cast<long long>(plan->row_blocks), kUsableCounters);
    plan->k_split = k_split;
    plan->chunk_groups = static_cast<int>(G / k_split);
    const size_t group_bytes = static_cast<size_t>(plan->staged_rows) * kDirectStride * sizeof(_Float16);
    int window = static_cast<int>(kDirectLdsBytes / group_bytes);
    // Windows of 34.8 KiB of activations: three workgroups per CU, and the
    // window fits the register staging. 32 staged rows: 4 groups, measured on
    // MI355X at M=17-32 gate/up 19.2-20.7 us against 26.2-26.9 in 8-group
    // windows, down 20.7-22.5 against 27.5-28.8, QKV and O 13.7-15.5 against
    // 15.3-17.1. Two tiles (64 staged rows): 2 groups, at M=40-64 gate/up
    // 31.6-32.8 us against 38.2-39.5 in 4-group windows with two workgroups
    // per CU (and 53.0 at M=40 in 8-group windows, one per CU), down
    // 33.7-35.5 against 40.7-43.1, QKV and O 23.2-25.9 against 24.9-27.2.
    if (plan->staged_rows == 32 && window > 4) window = 4;
    if (plan->nb == 2 && window > 2) window = 2;
    if (window >= plan->chunk_groups)
        window = plan->chunk_groups;
    else if (window >= 8)
        window -= window % 8;
    plan->window = window;
    plan->lds_bytes = static_cast<size_t>(window) * group_bytes;
    // Partials of the real activation columns only (at most 32 per tile).
    plan->partial_bytes = k_split > 1 ? static_cast<size_t>(k_split) * plan->row_blocks * kDirectRows *
                                            std::min<int64_t>(M, 32) * plan->nb * sizeof(float)
                                      : 0;
    return TERNEL_TQ1_OK;
}

template <int NB, int SR>
int launch_direct_kernel(const uint32_t *packed, const void *x, void *y, int64_t M, int64_t rows, int G,
                         const DirectPlan &plan, float *partial, unsigned *counters, hipStream_t stream) {
    int rc = ensure_lds_attribute(reinterpret_cast<const void *>(&direct_gemm_kernel<NB, SR>), kDirectLdsBytes);
    if (rc != TERNEL_TQ1_OK) return rc;
    const dim3 grid(static_cast<unsigned>(plan.row_blocks), static_cast<unsigned>(plan.k_split));
    hipLaunchKernelGGL((direct_gemm_kernel<NB, SR>), grid, dim3(kDirectThreads), plan.lds_bytes, stream, packed,
                       static_cast<const _Float16 *>(x), static_cast<_Float16 *>(y), partial, counters,
                       static_cast<int>(M), static_cast<int>(rows), G, plan.chunk_groups, plan.k_split, plan.window);
    TQ1_LAUNCH_CHECK();
    return TERNEL_TQ1_OK;
}

int launch_direct(const uint32_t *packed, const void *x, void *y, int64_t M, int64_t rows, int64_t columns,
                  const DirectPlan &plan, void *ws, hipStream_t stream) {
    unsigned *counters = plan.k_split > 1 ? static_cast<unsigned *>(ws) : nullptr;
    float *partial =
        plan.k_split > 1 ? reinterpret_cast<float *>(static_cast<char *>(ws) + kPartialOffset) : nullptr;
    const int G = static_cast<int>(columns / kBlockWeights);
    switch (plan.staged_rows) {
        case 8: return launch_direct_kernel<1, 8>(packed, x, y, M, rows, G, plan, partial, counters, stream);
        case 16: return launch_direct_kernel<1, 16>(packed, x, y, M, rows, G, plan, partial, counters, stream);
        case 32: return launch_direct_kernel<1, 32>(packed, x, y, M, rows, G, plan, partial, counters, stream);
        default: return launch_direct_kernel<2, 64>(packed, x, y, M, rows, G, plan, partial, counters, stream);
    }
}

// Wide form: stream-K over one workgroup per CU. Buffer resources address one
// activation tile (up to 256 rows) and one weight row tile (4 packed 64-row
// blocks) with 32-bit byte offsets.
constexpr int64_t kWideMaxColumns = INT32_MAX / (kWideMaxCols * 2) / kBlockWeights * kBlockWeights;

// Tile width (32-row activation blocks): the narrowest of 1, 2, 4, 8 that holds
// the batch, so small batches do not compute empty columns -- but 128-wide
// rather than 256-wide tiles where the stream-K reduction would weigh on a
// short loop.  A split tile's last contributor reads the other contributors'
// partials, about cus/tiles - 1 of them at tile size each, after a loop of
// tiles*groups/cus steps; 128-wide tiles halve the partial and, with twice the
// tiles, the contributors.  Take them while (cus/tiles - 1) / (tiles*groups/cus)
// exceeds 0.1.  Measured on MI355X (TFLOP/s, 256- / 128-wide tiles): down
// 17408->5120 M=256 375 / 550, M=512 694 / 775, M=768 835 / 841, M=1024
// 915 / 877; gate/up 5120->17408 M=256 559 / 687, M=512 865 / 824, M=768
// 928 / 861.
int wide_blocks(int64_t M, int64_t tiles_n, int64_t groups, int64_t cus) {
    const int nb = M <= 32 ? 1 : (M <= 64 ? 2 : (M <= 128 ? 4 : 8));
    const int64_t tiles = tiles_n * ceil_div(M, 256);
    return nb == 8 && 10 * (cus - tiles) * cus > tiles * tiles * groups ? 4 : nb;
}
int device_cu_count() {
    int dev = 0, cus = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0)
        return 256;
    return cus;
}

struct WidePlan {
    WideGeometry geo;
    int nb;  // tile width in 32-row activation blocks
    int workgroups;
    size_t partial_bytes;
    size_t xp_bytes;
};

int plan_wide(int64_t M, int64_t rows, int64_t columns, int k_split, WidePlan *plan) {
    if (k_split > 1)
        return fail(TERNEL_TQ1_EINVAL, "the wide form splits K by stream-K; k split must be 0 or 1, got %d", k_split);
    if (k_split < 0) return fail(TERNEL_TQ1_EINVAL, "k split must be positive, got %d", k_split);
    if (columns > kWideMaxColumns)
        return fail(TERNEL_TQ1_EINVAL, "the wide form takes at most %lld columns, got %lld",
                    static_cast<long long>(kWideMaxColumns), static_cast<long long>(columns));
    WideGeometry &g = plan->geo;
    g.M = static_cast<int>(M);
    g.N = static_cast<int>(rows);
    g.G = static_cast<int>(columns / kBlockWeights);
    g.row_blocks = static_cast<int>(ceil_div(rows, kTileRows));
    g.tiles_n = static_cast<int>(ceil_div(rows, kWideRows));
    plan->nb = wide_blocks(M, g.tiles_n, g.G, device_cu_count());
    const int64_t tiles = g.tiles_n * ceil_div(M, 32 * plan->nb);
    static_assert(2 * kWideTileSlots <= kUsableCounters, "two counters per wide tile");
    if (tiles > kWideTileSlots)
        return fail(TERNEL_TQ1_EINVAL, "%lld output tiles exceed the %d stream-K counters", static_cast<long long>(tiles),
                    kWideTileSlots);
    g.tiles = static_cast<int>(tiles);
    g.units = static_cast<int>(tiles * g.G);  // < 2^14 tiles x 2^15 groups
    g.vector_rows = 0;                         // set at launch from the output pointer
    g.spin_limit = g_spin_limit.load();
    int64_t wgs = device_cu_count();
    if (wgs > g.units) wgs = g.units;
    plan->workgroups = static_cast<int>(wgs);
    // two partial slots per workgroup, each all of its waves' accumulators
    plan->partial_bytes = static_cast<size_t>(wgs) * 2 * kWideWaves * wide_frag_floats(plan->nb) * sizeof(float);
    // the fp16 copy of the activations follows the partials (permuted for four
    // or eight blocks; one or two blocks read fp16 x itself and use the copy
    // for bf16 only), then bf16 rows' inverse scales
    plan->xp_bytes = static_cast<size_t>(M) * columns * sizeof(_Float16) + (M * sizeof(float) + 255) / 256 * 256;
    return TERNEL_TQ1_OK;
}

template <int NB, bool BF>
int launch_wide_kernel(const uint32_t *packed, const _Float16 *xp, void *y, float *partial, unsigned *counters,
                       const float *row_inv, const WideGeometry &geo, int workgroups, hipStream_t stream) {
    int rc = ensure_lds_attribute(reinterpret_cast<const void *>(&wide_gemm_kernel<NB, BF>),
                                  static_cast<int>(wide_lds_bytes(NB)));
    if (rc != TERNEL_TQ1_OK) return rc;
    hipLaunchKernelGGL((wide_gemm_kernel<NB, BF>), dim3(static_cast<unsigned>(workgroups)), dim3(kWideThreads),
                       wide_lds_bytes(NB), stream, packed, xp, static_cast<uint16_t *>(y), partial, counters, row_inv,
                       geo);
    TQ1_LAUNCH_CHECK();
    return TERNEL_TQ1_OK;
}

template <bool BF>
int launch_wide_nb(const uint32_t *packed, const _Float16 *xp, void *y, float *partial, unsigned *counters,
                   const float *row_inv, const WidePlan &plan, const WideGeometry &geo, hipStream_t stream) {
    switch (plan.nb) {
        case 1:
            return launch_wide_kernel<1, BF>(packed, xp, y, partial, counters, row_inv, geo, plan.workgroups, stream);
        case 2:
            return launch_wide_kernel<2, BF>(packed, xp, y, partial, counters, row_inv, geo, plan.workgroups, stream);
        case 4:
            return launch_wide_kernel<4, BF>(packed, xp, y, partial, counters, row_inv, geo, plan.workgroups, stream);
        default:
            return launch_wide_kernel<8, BF>(packed, xp, y, partial, counters, row_inv, geo, plan.workgroups, stream);
    }
}

int launch_wide(const uint32_t *packed, const void *x, void *y, const WidePlan &plan, void *ws, hipStream_t stream,
                int dtype) {
    unsigned *counters = static_cast<unsigned *>(ws);
    float *partial = reinterpret_cast<float *>(static_cast<char *>(ws) + kPartialOffset);
    _Float16 *copy = reinterpret_cast<_Float16 *>(static_cast<char *>(ws) + kPartialOffset + plan.partial_bytes);
    WideGeometry geo = plan.geo;
    geo.vector_rows = geo.N % 8 == 0 && reinterpret_cast<uintptr_t>(y) % 16 == 0;
    if (dtype == TERNEL_TQ1_BF16) {
        float *row_inv = reinterpret_cast<float *>(copy + static_cast<int64_t>(geo.M) * geo.G * kBlockWeights);
        const int64_t K = static_cast<int64_t>(geo.G) * kBlockWeights;
        if (plan.nb > 2)
            hipLaunchKernelGGL(scale_rows_kernel<true>, dim3(static_cast<unsigned>(geo.M)), dim3(kThreads), 0, stream,
                               static_cast<const uint16_t *>(x), copy, row_inv, K);
        else
            hipLaunchKernelGGL(scale_rows_kernel<false>, dim3(static_cast<unsigned>(geo.M)), dim3(kThreads), 0, stream,
                               static_cast<const uint16_t *>(x), copy, row_inv, K);
        TQ1_LAUNCH_CHECK();
        return launch_wide_nb<true>(packed, copy, y, partial, counters, row_inv, plan, geo, stream);
    }
    const _Float16 *xp = static_cast<const _Float16 *>(x);
    if (plan.nb > 2) {
        const int64_t quads = static_cast<int64_t>(plan.geo.M) * plan.geo.G * 8;  // 32-byte runs of the copy
        hipLaunchKernelGGL(permute_activations_kernel, dim3(static_cast<unsigned>(ceil_div(quads, kThreads))),
                           dim3(kThreads), 0, stream, static_cast<const uint2 *>(x), reinterpret_cast<uint2 *>(copy),
                           quads, static_cast<int>(reinterpret_cast<uintptr_t>(copy) % 16 == 0));
        TQ1_LAUNCH_CHECK();
        xp = copy;
    }
    return launch_wide_nb<false>(packed, xp, y, partial, counters, nullptr, plan, geo, stream);
}

// Automatic choice, from a sweep of every form over the 27B linears on MI355X
// (the fixture tests/golden/dispatch_sweep_mi355x.json replays it): the direct
// form up to 32 activation rows (gate/up, down M=24-32: 19.9-23.6 us against
// the wide form's 24.1-28.0; QKV, O 15.0-16.3 against 20.8-21.5), and up to
// 48 for matrices under 16 MiB of packed weights (QKV M=40-48: 22.2-23.0
// against 24.3-24.5; O 25.2-27.0 against 27.0-27.3); the wide form otherwise
// up to 64 rows (gate/up, down M=40-64: 28.9-33.6 against the two-tile direct
// form's 31.2-37.5; QKV and O at M=64 within 5 %); above, the wide form when
// stream-K has enough tiles or enough work per CU to amortise its reduction --
// at least CUs/4 tiles (a tile's partials come from at most ~4 contributors)
// or 15 (tile, group) steps per CU -- and the fixed-split tile form otherwise
// (QKV 5120->8192 M=128: 31.6 us against 38.8; gate/up 5120->17408 M=128: 44.6
// against 58.1 the other way). The tile form also serves a fixed K split above
// 32 rows and rows too long for the wide form's 32-bit buffer offsets.
constexpr int64_t kAutoDirectMaxBatch = 32;
constexpr int64_t kAutoDirectMaxBatchSmall = 48;
constexpr int64_t kAutoSmallMatrixBytes = 16ll << 20;
constexpr int64_t kAutoWideMaxBatch = 64;
int wide_blocks(int64_t M, int64_t tiles_n, int64_t groups, int64_t cus);
int device_cu_count();
int resolve_gemm_form(int64_t M, int64_t rows, int64_t columns, int form, int k_split) {
    if (form != TERNEL_TQ1_GEMM_AUTO) return form;
    const bool small = rows * (columns / kBlockWeights) * kBlockBytes < kAutoSmallMatrixBytes;
    if (M <= kAutoDirectMaxBatch || (small && M <= kAutoDirectMaxBatchSmall)) return TERNEL_TQ1_GEMM_DIRECT;
    const bool wide_ok = k_split <= 1 && columns <= kWideMaxColumns;
    if (M <= kAutoWideMaxBatch && wide_ok) return TERNEL_TQ1_GEMM_WIDE;
    if (k_split > 1 || columns > kWideMaxColumns) return TERNEL_TQ1_GEMM_TILE;
    const int64_t cus = device_cu_count();
    const int64_t groups = columns / kBlockWeights;
    const int64_t tiles_n = ceil_div(rows, kWideRows);
    const int nb = wide_blocks(M, tiles_n, groups, cus);
    const int64_t tiles = tiles_n * ceil_div(M, 32 * nb);
    // Measured on MI355X: above 64 rows (four or eight blocks per tile) 15
    // (tile, group) steps per CU (down M=96-128 stays on the tile form,
    // 49.6-52.4 us against 51.6-54.4).
    const int64_t min_steps = 15;
    return 4 * tiles >= cus || tiles * groups >= min_steps * cus ? TERNEL_TQ1_GEMM_WIDE : TERNEL_TQ1_GEMM_TILE;
}

// The dispatch rule of packed_matmul, retuned for MI355X by the same sweep: the
// LUT23 kernel up to 3 activation rows -- 4 for matrices under 16 MiB of
// packed weights, where the MFMA forms' fixed costs weigh more (O 8192->5120
// M=4: 11.5 us against the direct form's 13.1, M=5 13.7 against 13.0; gate/up
// M=4: the direct form 16.2 us against 18.9) -- the MFMA kernels above it
// (fp16 only).
constexpr int64_t kLinearLutMaxBatch = 3;
constexpr int64_t kLinearLutMaxBatchSmall = 4;
constexpr int64_t kLinearSmallMatrixBytes = 16ll << 20;
// bf16 activations above the same batch run the wide form (scale_rows_kernel
// then wide_gemm_kernel<NB, true>); fp32 ones always run the LUT23 kernel:
// their 24-bit significands do not fit the matrix cores' fp16 operands.
bool linear_uses_lut(int64_t M, int64_t rows, int64_t columns, int dtype) {
    if (dtype == TERNEL_TQ1_F32) return true;
    const int64_t bytes = rows * (columns / kBlockWeights) * kBlockBytes;
    return M <= (bytes < kLinearSmallMatrixBytes ? kLinearLutMaxBatchSmall : kLinearLutMaxBatch);
}

// The GEMM form of the library's dispatch for a batch that does not take the
// LUT23 kernel: bf16 activations run the wide form.
int linear_gemm_form(int64_t M, int64_t rows, int64_t columns, int dtype) {
    return dtype == TERNEL_TQ1_BF16 ? TERNEL_TQ1_GEMM_WIDE : TERNEL_TQ1_GEMM_AUTO;
}

int check_packed_pointer(const void *packed) {
    if (!packed) return fail(TERNEL_TQ1_EINVAL, "null pointer");
    if (reinterpret_cast<uintptr_t>(packed) & 3u) return fail(TERNEL_TQ1_EINVAL, "packed weights must be 4-byte aligned");
    return TERNEL_TQ1_OK;
}

}  // namespace

// ---------------------------------------------------------------------------
// C ABI
// ---------------------------------------------------------------------------
template <bool CANON>
int launch_get_rows(const uint32_t *table, int64_t rows, int64_t columns, const int64_t *ids, int64_t n_ids,
                    void *out, int dtype, void *stream) {
    g_last_error[0] = '\0';
    int rc;
    if ((rc = check_geometry(1, rows, columns)) != TERNEL_TQ1_OK) return rc;
    if ((rc = check_dtype(dtype)) != TERNEL_TQ1_OK) return rc;
    if (n_ids <= 0) return fail(TERNEL_TQ1_EINVAL, "indices are empty");
    if ((rc = check_packed_pointer(table)) != TERNEL_TQ1_OK) return rc;
    if (!ids || !out) return fail(TERNEL_TQ1_EINVAL, "null pointer");
    const int G = static_cast<int>(columns / kBlockWeights);
    if (n_ids > INT64_MAX / (static_cast<int64_t>(G) * kGatherRuns))
        return fail(TERNEL_TQ1_EINVAL, "too many indices for one gather");
    // Grid-stride over (token, group, run): at most 8 workgroups of 256 per CU
    // (an uncapped grid measured the same on MI355X: 8192 tokens 27.1 us
    // against 25.4).
    const int64_t threads = n_ids * G * kGatherRuns;
    const int64_t cap = static_cast<int64_t>(device_cu_count()) * 8;
    const dim3 grid(static_cast<unsigned>(std::min<int64_t>(ceil_div(threads, kThreads), cap)));
    const int vector_out = reinterpret_cast<uintptr_t>(out) % 16 == 0;
    hipStream_t s = static_cast<hipStream_t>(stream);
    switch (dtype) {
        case TERNEL_TQ1_F16:
            hipLaunchKernelGGL((get_rows_kernel<_Float16, CANON>), grid, dim3(kThreads), 0, s, table, rows, G, ids,
                               n_ids, static_cast<_Float16 *>(out), vector_out);
            break;
        case TERNEL_TQ1_BF16:
            hipLaunchKernelGGL((get_rows_kernel<bf16_t, CANON>), grid, dim3(kThreads), 0, s, table, rows, G, ids,
                               n_ids, static_cast<bf16_t *>(out), vector_out);
            break;
        default:
            hipLaunchKernelGGL((get_rows_kernel<float, CANON>), grid, dim3(kThreads), 0, s, table, rows, G, ids,
                               n_ids, static_cast<float *>(out), vector_out);
            break;
    }
    TQ1_LAUNCH_CHECK();
    return TERNEL_TQ1_OK;
}

// The split-K workspace of ternel_tq1_matmul_noalloc as a file-scope device
// array (counter region, then at most kNoAllocPartialBytes of fp32 partials),
// for callers that cannot allocate. Each device the library runs on holds its
// own copy until the process ends. In host code `scratch` is a stand-in, not
// a device address: kernels and copies only ever see the address resolved
// per device by noalloc_scratch().
constexpr int64_t kNoAllocPartialBytes = int64_t{16} << 20;
constexpr size_t kNoAllocScratchBytes = kPartialOffset + kNoAllocPartialBytes;
static __device__ __align__(256) unsigned scratch[kNoAllocScratchBytes / sizeof(unsigned)];

constexpr int kScratchDevices = 64;
std::mutex g_scratch_mutex;
void *g_scratch_address[kScratchDevices];  // per device; null until resolved

// This device's copy of `scratch`. The first call on a device resolves its
// address and zeroes its counter region on `stream` (stream-ordered before the
// launch that follows); the LUT23 fix-up leaves every counter it used at zero,
// so the region stays zero between calls. The set-up call may not be under
// stream capture.
int noalloc_scratch(hipStream_t stream, void **out) {
    int device = 0;
    hipError_t e = hipGetDevice(&device);
    if (e != hipSuccess) return fail(TERNEL_TQ1_EHIP, "hipGetDevice: %s", hipGetErrorString(e));
    if (device < 0 || device >= kScratchDevices)
        return fail(TERNEL_TQ1_EINVAL, "device %d is past the %d whose scratch addresses are kept", device,
                    kScratchDevices);
    std::lock_guard<std::mutex> lock(g_scratch_mutex);
    if (!g_scratch_address[device]) {
        hipStreamCaptureStatus capture = hipStreamCaptureStatusNone;
        if ((e = hipStreamIsCapturing(stream, &capture)) != hipSuccess)
            return fail(TERNEL_TQ1_EHIP, "hipStreamIsCapturing: %s", hipGetErrorString(e));
        if (capture != hipStreamCaptureStatusNone)
            return fail(TERNEL_TQ1_EINVAL,
                        "the first ternel_tq1_matmul_noalloc call on device %d is under stream capture; make one "
                        "call outside capture first (it sets up the device's scratch)",
                        device);
        void *address = nullptr;
        if ((e = hipGetSymbolAddress(&address, HIP_SYMBOL(scratch))) != hipSuccess)
            return fail(TERNEL_TQ1_EHIP, "resolving the scratch array on device %d: %s", device,
                        hipGetErrorString(e));
        if ((e = hipMemsetAsync(address, 0, kCounterRegionBytes, stream)) != hipSuccess)
            return fail(TERNEL_TQ1_EHIP, "clearing the scratch counters: %s", hipGetErrorString(e));
        g_scratch_address[device] = address;
    }
    *out = g_scratch_address[device];
    return TERNEL_TQ1_OK;
}

extern "C" {

const char *ternel_tq1_last_error(void) { return g_last_error; }

const char *ternel_tq1_version(void) { return "ternel-tq1-gfx950 0.3.0"; }

int ternel_tq1_workspace_error(const void *ws, size_t ws_bytes, int *error, void *stream) {
    g_last_error[0] = '\0';
    if (!ws || !error) return fail(TERNEL_TQ1_EINVAL, "null pointer");
    if (ws_bytes < kCounterRegionBytes)
        return fail(TERNEL_TQ1_EINVAL, "workspace of %zu bytes has no error word", ws_bytes);
    unsigned word = 0;
    hipStream_t s = static_cast<hipStream_t>(stream);
    hipError_t e = hipMemcpyAsync(&word, static_cast<const unsigned *>(ws) + kErrorSlot, sizeof(word),
                                  hipMemcpyDeviceToHost, s);
    if (e == hipSuccess) e = hipStreamSynchronize(s);
    if (e != hipSuccess) return fail(TERNEL_TQ1_EHIP, "reading the workspace error word: %s", hipGetErrorString(e));
    *error = static_cast<int>(word);
    return TERNEL_TQ1_OK;
}

#ifdef TERNEL_TQ1_PROFILE
// Profile build only: copies (synchronously) and clears the phase stamps of
// the last stream-GEMV launches; returns the number of waves copied.
int ternel_tq1_profile_stamps(unsigned long long *host, int64_t max_waves, void *stream) {
    const int64_t waves = max_waves < kPhaseWaves ? max_waves : kPhaseWaves;
    hipStream_t s = static_cast<hipStream_t>(stream);
    hipError_t e = hipStreamSynchronize(s);
    if (e == hipSuccess)
        e = hipMemcpyFromSymbol(host, HIP_SYMBOL(g_phase_stamps), waves * kPhaseSlots * sizeof(unsigned long long), 0,
                                hipMemcpyDeviceToHost);
    static unsigned long long zeros[kPhaseWaves][kPhaseSlots];
    if (e == hipSuccess) e = hipMemcpyToSymbol(HIP_SYMBOL(g_phase_stamps), zeros, sizeof(zeros), 0, hipMemcpyHostToDevice);
    if (e != hipSuccess) return fail(TERNEL_TQ1_EHIP, "phase stamps: %s", hipGetErrorString(e));
    return static_cast<int>(waves);
}
#endif

int ternel_tq1_set_spin_limit(int limit) {
    const int old = g_spin_limit.load();
    g_spin_limit.store(limit);
    return old;
}

int64_t ternel_tq1_packed_words(int64_t rows, int64_t columns) {
    if (rows <= 0 || columns <= 0 || columns % kBlockWeights) return 0;
    return packed_words(rows, columns);
}

int ternel_tq1_validate(const uint8_t *blocks, int64_t nblocks, uint64_t *counters, void *stream) {
    g_last_error[0] = '\0';
    if (!counters) return fail(TERNEL_TQ1_EINVAL, "null pointer");
    if (nblocks < 0) return fail(TERNEL_TQ1_EINVAL, "negative block count");
    if (nblocks > 0 && !blocks) return fail(TERNEL_TQ1_EINVAL, "null pointer");
    if (reinterpret_cast<uintptr_t>(blocks) & 3u) return fail(TERNEL_TQ1_EINVAL, "blocks must be 4-byte aligned");
    hipStream_t s = static_cast<hipStream_t>(stream);
    auto *cnt = reinterpret_cast<unsigned long long *>(counters);
    hipLaunchKernelGGL(zero_u64_kernel, dim3(1), dim3(64), 0, s, cnt, 2);
    TQ1_LAUNCH_CHECK();
    if (nblocks == 0) return TERNEL_TQ1_OK;
    const int64_t nwords = nblocks * kBlockWords;
    int64_t grid = ceil_div(nwords, kThreads * 4);
    if (grid > 8192) grid = 8192;
    hipLaunchKernelGGL(validate_kernel, dim3(static_cast<unsigned>(grid)), dim3(kThreads), 0, s,
                       reinterpret_cast<const uint32_t *>(blocks), nwords, cnt);
    TQ1_LAUNCH_CHECK();
    return TERNEL_TQ1_OK;
}

int ternel_tq1_from_q2(const uint8_t *q2_blocks, int64_t nblocks, uint8_t *blocks, uint64_t *bad_codes,
                       void *stream) {
    g_last_error[0] = '\0';
    if (!bad_codes) return fail(TERNEL_TQ1_EINVAL, "null pointer");
    if (nblocks < 0) return fail(TERNEL_TQ1_EINVAL, "negative block count");
    if (nblocks > 0 && (!q2_blocks || !blocks)) return fail(TERNEL_TQ1_EINVAL, "null pointer");
    if (nblocks > INT64_MAX / kQ2Slots) return fail(TERNEL_TQ1_EINVAL, "too many blocks");
    hipStream_t s = static_cast<hipStream_t>(stream);
    auto *cnt = reinterpret_cast<unsigned long long *>(bad_codes);
    hipLaunchKernelGGL(zero_u64_kernel, dim3(1), dim3(64), 0, s, cnt, 1);
    TQ1_LAUNCH_CHECK();
    if (nblocks == 0) return TERNEL_TQ1_OK;
    int64_t grid = ceil_div(nblocks * kQ2Slots, kThreads);
    if (grid > 65536) grid = 65536;
    hipLaunchKernelGGL(q2_to_tq1_kernel, dim3(static_cast<unsigned>(grid)), dim3(kThreads), 0, s, q2_blocks, blocks,
                       nblocks, cnt);
    TQ1_LAUNCH_CHECK();
    return TERNEL_TQ1_OK;
}

int ternel_tq1_decode(const uint8_t *blocks, int64_t nblocks, uint8_t *scales_out, uint8_t *codes_out,
                      void *stream) {
    g_last_error[0] = '\0';
    if (nblocks < 0) return fail(TERNEL_TQ1_EINVAL, "negative block count");
    if (nblocks == 0) return TERNEL_TQ1_OK;
    if (!blocks || !scales_out || !codes_out) return fail(TERNEL_TQ1_EINVAL, "null pointer");
    const int64_t grid = ceil_div(nblocks * kCodeSlots, kThreads);
    if (grid > INT32_MAX) return fail(TERNEL_TQ1_EINVAL, "too many blocks for one decode launch");
    hipLaunchKernelGGL(decode_kernel, dim3(static_cast<unsigned>(grid)), dim3(kThreads), 0,
                       static_cast<hipStream_t>(stream), blocks, nblocks, scales_out, codes_out);
    TQ1_LAUNCH_CHECK();
    return TERNEL_TQ1_OK;
}

int ternel_tq1_interleave(const uint8_t *blocks, int64_t rows, int64_t columns, uint32_t *packed, void *stream) {
    g_last_error[0] = '\0';
    int rc;
    if ((rc = check_geometry(1, rows, columns)) != TERNEL_TQ1_OK) return rc;
    if (!blocks || !packed) return fail(TERNEL_TQ1_EINVAL, "null pointer");
    if ((reinterpret_cast<uintptr_t>(blocks) | reinterpret_cast<uintptr_t>(packed)) & 3u)
        return fail(TERNEL_TQ1_EINVAL, "blocks and packed weights must be 4-byte aligned");
    const int64_t total = packed_words(rows, columns);
    hipLaunchKernelGGL(interleave_kernel, dim3(static_cast<unsigned>(ceil_div(total, kThreads))), dim3(kThreads), 0,
                       static_cast<hipStream_t>(stream), reinterpret_cast<const uint32_t *>(blocks), packed, rows,
                       columns / kBlockWeights, total);
    TQ1_LAUNCH_CHECK();
    return TERNEL_TQ1_OK;
}

static int check_tiled(int64_t rows, int64_t columns, int64_t tile) {
    int rc;
    if ((rc = check_geometry(1, rows, columns)) != TERNEL_TQ1_OK) return rc;
    if (tile <= 0 || rows % tile)
        return fail(TERNEL_TQ1_EINVAL, "tile %lld does not divide the tensor's %lld rows", static_cast<long long>(tile),
                    static_cast<long long>(rows));
    return TERNEL_TQ1_OK;
}

int ternel_tq1_words_from_tiled(const uint8_t *codes, const uint16_t *scales, int64_t rows, int64_t columns,
                                int64_t tile, uint32_t *packed, uint64_t *counters, void *stream) {
    g_last_error[0] = '\0';
    int rc;
    if ((rc = check_tiled(rows, columns, tile)) != TERNEL_TQ1_OK) return rc;
    if (!codes || !scales || !packed || !counters) return fail(TERNEL_TQ1_EINVAL, "null pointer");
    if ((reinterpret_cast<uintptr_t>(scales) & 1u) || (reinterpret_cast<uintptr_t>(packed) & 3u))
        return fail(TERNEL_TQ1_EINVAL, "scales must be 2-byte and packed words 4-byte aligned");
    hipStream_t s = static_cast<hipStream_t>(stream);
    auto *cnt = reinterpret_cast<unsigned long long *>(counters);
    hipLaunchKernelGGL(zero_u64_kernel, dim3(1), dim3(64), 0, s, cnt, 2);
    TQ1_LAUNCH_CHECK();
    const int64_t total = packed_words(rows, columns);
    hipLaunchKernelGGL(words_from_tiled_kernel, dim3(static_cast<unsigned>(ceil_div(total, kThreads))), dim3(kThreads),
                       0, s, codes, scales, packed, rows, columns / kBlockWeights, tile, total, cnt);
    TQ1_LAUNCH_CHECK();
    return TERNEL_TQ1_OK;
}

int ternel_tq1_tiled_from_words(const uint32_t *packed, int64_t rows, int64_t columns, int64_t tile, uint8_t *codes,
                                uint16_t *scales, void *stream) {
    g_last_error[0] = '\0';
    int rc;
    if ((rc = check_tiled(rows, columns, tile)) != TERNEL_TQ1_OK) return rc;
    if (!codes || !scales || !packed) return fail(TERNEL_TQ1_EINVAL, "null pointer");
    if ((reinterpret_cast<uintptr_t>(scales) & 1u) || (reinterpret_cast<uintptr_t>(packed) & 3u))
        return fail(TERNEL_TQ1_EINVAL, "scales must be 2-byte and packed words 4-byte aligned");
    const int64_t total = packed_words(rows, columns);
    hipLaunchKernelGGL(tiled_from_words_kernel, dim3(static_cast<unsigned>(ceil_div(total, kThreads))), dim3(kThreads),
                       0, static_cast<hipStream_t>(stream), packed, codes, scales, rows, columns / kBlockWeights, tile,
                       total);
    TQ1_LAUNCH_CHECK();
    return TERNEL_TQ1_OK;
}

int ternel_tq1_deinterleave(const uint32_t *packed, int64_t rows, int64_t columns, uint8_t *blocks, void *stream) {
    g_last_error[0] = '\0';
    int rc;
    if ((rc = check_geometry(1, rows, columns)) != TERNEL_TQ1_OK) return rc;
    if (!blocks || !packed) return fail(TERNEL_TQ1_EINVAL, "null pointer");
    if ((reinterpret_cast<uintptr_t>(blocks) | reinterpret_cast<uintptr_t>(packed)) & 3u)
        return fail(TERNEL_TQ1_EINVAL, "blocks and packed weights must be 4-byte aligned");
    const int64_t total = rows * (columns / kBlockWeights) * kBlockWords;
    hipLaunchKernelGGL(deinterleave_kernel, dim3(static_cast<unsigned>(ceil_div(total, kThreads))), dim3(kThreads),
                       0, static_cast<hipStream_t>(stream), packed, reinterpret_cast<uint32_t *>(blocks),
                       columns / kBlockWeights, total);
    TQ1_LAUNCH_CHECK();
    return TERNEL_TQ1_OK;
}

size_t ternel_tq1_matmul_workspace_bytes(int64_t M, int64_t rows, int64_t columns, int batch_tile, int k_split) {
    if (check_geometry(M, rows, columns) != TERNEL_TQ1_OK) return 0;
    if (uses_strip_gemv(M, batch_tile, k_split, rows, columns)) {
        StripGeometry geo;
        return plan_strip(rows, columns, &geo) == TERNEL_TQ1_OK ? strip_workspace_bytes(geo) : 0;
    }
    LutPlan plan;
    if (plan_lut(M, rows, columns, batch_tile, k_split, &plan) != TERNEL_TQ1_OK) return 0;
    return plan.counter_bytes + plan.partial_bytes;
}

int ternel_tq1_matmul(const uint32_t *packed, const void *x, void *y, int64_t M, int64_t rows, int64_t columns,
                      int dtype, int batch_tile, int k_split, void *ws, size_t ws_bytes, void *stream) {
    g_last_error[0] = '\0';
    int rc;
    if ((rc = check_geometry(M, rows, columns)) != TERNEL_TQ1_OK) return rc;
    if ((rc = check_dtype(dtype)) != TERNEL_TQ1_OK) return rc;
    if (uses_strip_gemv(M, batch_tile, k_split, rows, columns)) {
        StripGeometry geo;
        if ((rc = plan_strip(rows, columns, &geo)) != TERNEL_TQ1_OK) return rc;
        if ((rc = check_packed_pointer(packed)) != TERNEL_TQ1_OK) return rc;
        if (!x || !y) return fail(TERNEL_TQ1_EINVAL, "null pointer");
        const size_t need = strip_workspace_bytes(geo);
        if (need && (!ws || ws_bytes < need))
            return fail(TERNEL_TQ1_EINVAL, "workspace of %zu bytes is smaller than the %zu the split needs", ws_bytes,
                        need);
        hipStream_t s = static_cast<hipStream_t>(stream);
        switch (dtype) {
            case TERNEL_TQ1_F16:
                return launch_strip<_Float16>(packed, x, y, geo, s, false, ws);
            case TERNEL_TQ1_BF16:
                return launch_strip<bf16_t>(packed, x, y, geo, s, false, ws);
            default:
                return launch_strip<float>(packed, x, y, geo, s, false, ws);
        }
    }
    LutPlan plan;
    if ((rc = plan_lut(M, rows, columns, batch_tile, k_split, &plan)) != TERNEL_TQ1_OK) return rc;
    if ((rc = check_packed_pointer(packed)) != TERNEL_TQ1_OK) return rc;
    if (!x || !y) return fail(TERNEL_TQ1_EINVAL, "null pointer");
    const size_t need = plan.counter_bytes + plan.partial_bytes;
    if (need && (!ws || ws_bytes < need))
        return fail(TERNEL_TQ1_EINVAL, "workspace of %zu bytes is smaller than the %zu the split needs", ws_bytes,
                    need);
    hipStream_t s = static_cast<hipStream_t>(stream);
    switch (dtype) {
        case TERNEL_TQ1_F16:
            return launch_lut<_Float16>(packed, x, y, M, rows, columns, plan, ws, s);
        case TERNEL_TQ1_BF16:
            return launch_lut<bf16_t>(packed, x, y, M, rows, columns, plan, ws, s);
        default:
            return launch_lut<float>(packed, x, y, M, rows, columns, plan, ws, s);
    }
}

int ternel_tq1_matmul_noalloc(const uint32_t *packed, const void *x, void *y, int64_t M, int64_t rows,
                              int64_t columns, int dtype, int batch_tile, int k_split, void *stream) {
    g_last_error[0] = '\0';
    int rc;
    if ((rc = check_geometry(M, rows, columns)) != TERNEL_TQ1_OK) return rc;
    if ((rc = check_dtype(dtype)) != TERNEL_TQ1_OK) return rc;
    if (uses_strip_gemv(M, batch_tile, k_split, rows, columns)) {
        // the same kernel as ternel_tq1_matmul; a split one meets its K
        // chunks in the static scratch's counter region
        StripGeometry geo;
        if ((rc = plan_strip(rows, columns, &geo)) != TERNEL_TQ1_OK) return rc;
        if ((rc = check_packed_pointer(packed)) != TERNEL_TQ1_OK) return rc;
        if (!x || !y) return fail(TERNEL_TQ1_EINVAL, "null pointer");
        hipStream_t s = static_cast<hipStream_t>(stream);
        void *ws = nullptr;
        if (geo.Z > 1 && (rc = noalloc_scratch(s, &ws)) != TERNEL_TQ1_OK) return rc;
        switch (dtype) {
            case TERNEL_TQ1_F16:
                return launch_strip<_Float16>(packed, x, y, geo, s, false, ws);
            case TERNEL_TQ1_BF16:
                return launch_strip<bf16_t>(packed, x, y, geo, s, false, ws);
            default:
                return launch_strip<float>(packed, x, y, geo, s, false, ws);
        }
    }
    LutPlan plan;
    if ((rc = plan_lut(M, rows, columns, batch_tile, k_split, &plan, kNoAllocPartialBytes)) != TERNEL_TQ1_OK)
        return rc;
    if (plan.partial_bytes > static_cast<size_t>(kNoAllocPartialBytes))
        return fail(TERNEL_TQ1_EINVAL,
                    "a k split of %d over %lld rows needs %lld bytes of partials per batch tile of %d, more than "
                    "the %lld bytes of the static scratch",
                    plan.k_split, static_cast<long long>(rows),
                    static_cast<long long>(plan.k_split) * plan.batch_tile * rows * static_cast<long long>(sizeof(float)),
                    plan.batch_tile, static_cast<long long>(kNoAllocPartialBytes));
    if ((rc = check_packed_pointer(packed)) != TERNEL_TQ1_OK) return rc;
    if (!x || !y) return fail(TERNEL_TQ1_EINVAL, "null pointer");
    hipStream_t s = static_cast<hipStream_t>(stream);
    void *ws = nullptr;
    if (plan.k_split > 1 && (rc = noalloc_scratch(s, &ws)) != TERNEL_TQ1_OK) return rc;
    switch (dtype) {
        case TERNEL_TQ1_F16:
            return launch_lut<_Float16>(packed, x, y, M, rows, columns, plan, ws, s);
        case TERNEL_TQ1_BF16:
            return launch_lut<bf16_t>(packed, x, y, M, rows, columns, plan, ws, s);
        default:
            return launch_lut<float>(packed, x, y, M, rows, columns, plan, ws, s);
    }
}

size_t ternel_tq1_gemm_workspace_bytes(int64_t M, int64_t rows, int64_t columns, int form, int k_split) {
    if (check_geometry(M, rows, columns) != TERNEL_TQ1_OK) return 0;
    form = resolve_gemm_form(M, rows, columns, form, k_split);
    if (form == TERNEL_TQ1_GEMM_DIRECT) {
        DirectPlan direct;
        if (plan_direct(M, rows, columns, k_split, &direct) != TERNEL_TQ1_OK) return 0;
        return direct.k_split > 1 ? kPartialOffset + direct.partial_bytes : 0;
    }
    if (form == TERNEL_TQ1_GEMM_WIDE) {
        WidePlan wide;
        if (plan_wide(M, rows, columns, k_split, &wide) != TERNEL_TQ1_OK) return 0;
        return kPartialOffset + wide.partial_bytes + wide.xp_bytes;
    }
    if (form != TERNEL_TQ1_GEMM_TILE) return 0;
    GemmPlan plan;
    if (plan_gemm(M, rows, columns, k_split, &plan) != TERNEL_TQ1_OK) return 0;
    return plan.k_split > 1 ? kPartialOffset + static_cast<size_t>(plan.k_split) * M * rows * sizeof(float)
                            : 0;
}

int ternel_tq1_gemm(const uint32_t *packed, const void *x, void *y, int64_t M, int64_t rows, int64_t columns,
                    int dtype, int form, int k_split, void *ws, size_t ws_bytes, void *stream) {
    g_last_error[0] = '\0';
    int rc;
    if ((rc = check_geometry(M, rows, columns)) != TERNEL_TQ1_OK) return rc;
    if (dtype != TERNEL_TQ1_F16 && dtype != TERNEL_TQ1_BF16)
        return fail(TERNEL_TQ1_EINVAL, "the MFMA path takes fp16 or bf16 activations, got dtype code %d", dtype);
    if (form != TERNEL_TQ1_GEMM_AUTO && form != TERNEL_TQ1_GEMM_TILE && form != TERNEL_TQ1_GEMM_DIRECT &&
        form != TERNEL_TQ1_GEMM_WIDE)
        return fail(TERNEL_TQ1_EINVAL, "unknown GEMM form %d", form);
    if (dtype == TERNEL_TQ1_BF16) {
        if (form != TERNEL_TQ1_GEMM_AUTO && form != TERNEL_TQ1_GEMM_WIDE)
            return fail(TERNEL_TQ1_EINVAL, "bf16 activations run the wide form (form %d or %d), got %d",
                        TERNEL_TQ1_GEMM_AUTO, TERNEL_TQ1_GEMM_WIDE, form);
        if (k_split > 1) return fail(TERNEL_TQ1_EINVAL, "the wide form takes no fixed K split, got %d", k_split);
        form = TERNEL_TQ1_GEMM_WIDE;
    }
    form = resolve_gemm_form(M, rows, columns, form, k_split);
    if (form == TERNEL_TQ1_GEMM_DIRECT) {
        DirectPlan direct;
        if ((rc = plan_direct(M, rows, columns, k_split, &direct)) != TERNEL_TQ1_OK) return rc;
        if ((rc = check_packed_pointer(packed)) != TERNEL_TQ1_OK) return rc;
        if (!x || !y) return fail(TERNEL_TQ1_EINVAL, "null pointer");
        if (reinterpret_cast<uintptr_t>(x) & 15u) return fail(TERNEL_TQ1_EINVAL, "activations must be 16-byte aligned");
        const size_t need = direct.k_split > 1 ? kPartialOffset + direct.partial_bytes : 0;
        if (need && (!ws || ws_bytes < need))
            return fail(TERNEL_TQ1_EINVAL, "workspace of %zu bytes is smaller than the %zu the split needs", ws_bytes,
                        need);
        return launch_direct(packed, x, y, M, rows, columns, direct, ws, static_cast<hipStream_t>(stream));
    }
    if (form == TERNEL_TQ1_GEMM_WIDE) {
        WidePlan wide;
        if ((rc = plan_wide(M, rows, columns, k_split, &wide)) != TERNEL_TQ1_OK) return rc;
        if ((rc = check_packed_pointer(packed)) != TERNEL_TQ1_OK) return rc;
        if (!x || !y) return fail(TERNEL_TQ1_EINVAL, "null pointer");
        if (reinterpret_cast<uintptr_t>(x) & 15u) return fail(TERNEL_TQ1_EINVAL, "activations must be 16-byte aligned");
        const size_t need = kPartialOffset + wide.partial_bytes + wide.xp_bytes;
        if (!ws || ws_bytes < need)
            return fail(TERNEL_TQ1_EINVAL, "workspace of %zu bytes is smaller than the %zu the split needs", ws_bytes,
                        need);
        return launch_wide(packed, x, y, wide, ws, static_cast<hipStream_t>(stream), dtype);
    }
    GemmPlan plan;
    if ((rc = plan_gemm(M, rows, columns, k_split, &plan)) != TERNEL_TQ1_OK) return rc;
    if ((rc = check_packed_pointer(packed)) != TERNEL_TQ1_OK) return rc;
    if (!x || !y) return fail(TERNEL_TQ1_EINVAL, "null pointer");
    if (reinterpret_cast<uintptr_t>(x) & 15u) return fail(TERNEL_TQ1_EINVAL, "activations must be 16-byte aligned");
    float *partial = nullptr;
    if (plan.k_split > 1) {
        // Partials go past the counter region, which stays untouched (and zero).
        const size_t need = kPartialOffset + static_cast<size_t>(plan.k_split) * M * rows * sizeof(float);
        if (!ws || ws_bytes < need)
            return fail(TERNEL_TQ1_EINVAL, "workspace of %zu bytes is smaller than the %zu the split needs", ws_bytes,
                        need);
        partial = reinterpret_cast<float *>(static_cast<char *>(ws) + kPartialOffset);
    }
    return launch_gemm(packed, x, y, M, rows, columns, plan, partial, static_cast<hipStream_t>(stream));
}

int ternel_tq1_get_rows(const uint32_t *packed, int64_t rows, int64_t columns, const int64_t *ids, int64_t n_ids,
                        void *out, int dtype, void *stream) {
    return launch_get_rows<false>(packed, rows, columns, ids, n_ids, out, dtype, stream);
}

int ternel_tq1_get_rows_canonical(const uint8_t *blocks, int64_t rows, int64_t columns, const int64_t *ids,
                                  int64_t n_ids, void *out, int dtype, void *stream) {
    if (reinterpret_cast<uintptr_t>(blocks) % 4)
        return fail(TERNEL_TQ1_EINVAL, "canonical blocks must be 4-byte aligned");
    return launch_get_rows<true>(reinterpret_cast<const uint32_t *>(blocks), rows, columns, ids, n_ids, out, dtype,
                                 stream);
}

size_t ternel_tq1_linear_workspace_bytes(int64_t M, int64_t rows, int64_t columns, int dtype) {
    if (linear_uses_lut(M, rows, columns, dtype))
        return ternel_tq1_matmul_workspace_bytes(M, rows, columns, 0, 0);
    return ternel_tq1_gemm_workspace_bytes(M, rows, columns, linear_gemm_form(M, rows, columns, dtype), 0);
}

int ternel_tq1_linear(const uint32_t *packed, const void *x, void *y, int64_t M, int64_t rows, int64_t columns,
                      int dtype, void *ws, size_t ws_bytes, void *stream) {
    if (linear_uses_lut(M, rows, columns, dtype))
        return ternel_tq1_matmul(packed, x, y, M, rows, columns, dtype, 0, 0, ws, ws_bytes, stream);
    return ternel_tq1_gemm(packed, x, y, M, rows, columns, dtype, linear_gemm_form(M, rows, columns, dtype), 0, ws,
                           ws_bytes, stream);
}

// Where the GEMM path's fp16 gate/up output sits in the workspace: after the
// GEMM's own workspace and never inside the counter region that every call
// expects to find zero.
static size_t swiglu_pairs_offset(int64_t M, int64_t rows, int64_t columns, int dtype) {
    const size_t gemm = ternel_tq1_gemm_workspace_bytes(M, rows, columns, linear_gemm_form(M, rows, columns, dtype), 0);
    return (std::max(gemm, kPartialOffset) + 255) / 256 * 256;
}

int ternel_tq1_linear_kernel(int64_t M, int64_t rows, int64_t columns, int dtype) {
    g_last_error[0] = '\0';
    int rc;
    if ((rc = check_geometry(M, rows, columns)) != TERNEL_TQ1_OK) return rc;
    if ((rc = check_dtype(dtype)) != TERNEL_TQ1_OK) return rc;
    if (linear_uses_lut(M, rows, columns, dtype)) return TERNEL_TQ1_KERNEL_LUT23;
    return resolve_gemm_form(M, rows, columns, linear_gemm_form(M, rows, columns, dtype), 0);
}

size_t ternel_tq1_swiglu_workspace_bytes(int64_t M, int64_t rows, int64_t columns, int dtype) {
    if (check_geometry(M, rows, columns) != TERNEL_TQ1_OK || rows % 2) return 0;
    if (linear_uses_lut(M, rows, columns, dtype))
        return ternel_tq1_matmul_workspace_bytes(M, rows, columns, uses_strip_gemv(M, 0, 0, rows, columns, false) ? 0 : 1,
                                                 0);
    return swiglu_pairs_offset(M, rows, columns, dtype) + static_cast<size_t>(M) * rows * sizeof(_Float16);
}

int ternel_tq1_swiglu(const uint32_t *packed, const void *x, void *z, int64_t M, int64_t rows, int64_t columns,
                      int dtype, void *ws, size_t ws_bytes, void *stream) {
    g_last_error[0] = '\0';
    int rc;
    if ((rc = check_geometry(M, rows, columns)) != TERNEL_TQ1_OK) return rc;
    if ((rc = check_dtype(dtype)) != TERNEL_TQ1_OK) return rc;
    if (rows % 2)
        return fail(TERNEL_TQ1_EINVAL, "a SwiGLU weight interleaves gate and up rows, so its rows must be even, got %lld",
                    static_cast<long long>(rows));
    if ((rc = check_packed_pointer(packed)) != TERNEL_TQ1_OK) return rc;
    if (!x || !z) return fail(TERNEL_TQ1_EINVAL, "null pointer");
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (linear_uses_lut(M, rows, columns, dtype) && uses_strip_gemv(M, 0, 0, rows, columns, false)) {
        StripGeometry geo;
        if ((rc = plan_strip(rows, columns, &geo, false)) != TERNEL_TQ1_OK) return rc;
        switch (dtype) {
            case TERNEL_TQ1_F16:
                return launch_strip<_Float16>(packed, x, z, geo, s, true);
            case TERNEL_TQ1_BF16:
                return launch_strip<bf16_t>(packed, x, z, geo, s, true);
            default:
                return launch_strip<float>(packed, x, z, geo, s, true);
        }
    }
    if (linear_uses_lut(M, rows, columns, dtype)) {
        LutPlan plan;
        if ((rc = plan_lut(M, rows, columns, 1, 0, &plan)) != TERNEL_TQ1_OK) return rc;
        const size_t need = plan.counter_bytes + plan.partial_bytes;
        if (need && (!ws || ws_bytes < need))
            return fail(TERNEL_TQ1_EINVAL, "workspace of %zu bytes is smaller than the %zu the split needs", ws_bytes,
                        need);
        switch (dtype) {
            case TERNEL_TQ1_F16:
                return launch_lut<_Float16>(packed, x, z, M, rows, columns, plan, ws, s, true);
            case TERNEL_TQ1_BF16:
                return launch_lut<bf16_t>(packed, x, z, M, rows, columns, plan, ws, s, true);
            default:
                return launch_lut<float>(packed, x, z, M, rows, columns, plan, ws, s, true);
        }
    }
    const size_t need = ternel_tq1_swiglu_workspace_bytes(M, rows, columns, dtype);
    if (need == 0 || !ws || ws_bytes < need)
        return fail(TERNEL_TQ1_EINVAL, "workspace of %zu bytes is smaller than the %zu a SwiGLU GEMM needs", ws_bytes,
                    need);
    const int gemm_form = linear_gemm_form(M, rows, columns, dtype);
    const size_t gemm = ternel_tq1_gemm_workspace_bytes(M, rows, columns, gemm_form, 0);
    void *pairs = static_cast<char *>(ws) + swiglu_pairs_offset(M, rows, columns, dtype);
    if ((rc = ternel_tq1_gemm(packed, x, pairs, M, rows, columns, dtype, gemm_form, 0, gemm ? ws : nullptr, gemm,
                              stream)) != TERNEL_TQ1_OK)
        return rc;
    const int64_t count = M * (rows / 2);
    int64_t grid = ceil_div(count, kThreads);
    if (grid > 65536) grid = 65536;
    if (dtype == TERNEL_TQ1_BF16)
        hipLaunchKernelGGL((swiglu_pairs_kernel<bf16_t>), dim3(static_cast<unsigned>(grid)), dim3(kThreads), 0, s,
                           static_cast<const bf16_t *>(pairs), static_cast<bf16_t *>(z), count);
    else
        hipLaunchKernelGGL((swiglu_pairs_kernel<_Float16>), dim3(static_cast<unsigned>(grid)), dim3(kThreads), 0, s,
                           static_cast<const _Float16 *>(pairs), static_cast<_Float16 *>(z), count);
    TQ1_LAUNCH_CHECK();
    return TERNEL_TQ1_OK;
}

}  // extern "C"
