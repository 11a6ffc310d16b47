// tq1_bytes.h -- the integer arithmetic the TQ1_G128 kernels apply to a code
// byte, and the geometry of the LUT23 tables it indexes.
//
// The kernels include this header (device), and so does the host-side check
// tests/byte_bounds.cpp, which walks every byte value 0..255, legal or not,
// through the same functions: for legal bytes (codes <= 242, tail <= 26) they
// give the exact base-3 digits, and for every byte value each table entry
// they select lies inside its group's table and each digit carrier holds a
// digit in 0..2. That is what keeps the compute kernels memory-safe on bytes
// that were never validated.
//
// Compiled by hipcc, where __host__ / __device__ are defined, or by a host
// compiler that defines them empty.
#ifndef TERNEL_TQ1_BYTES_H
#define TERNEL_TQ1_BYTES_H

#include <stdint.h>

namespace tq1_bytes {

// Block format (src/bonsai_tq1/format.py:14-24): 25 code bytes of five trits,
// then a tail byte of three.
constexpr int kFullSlots = 25;
constexpr uint32_t kMaxCodeByte = 242;
constexpr uint32_t kMaxTailByte = 26;

// LUT23 tables of one 128-weight group, fp32: L2[25][9] over trits (0,1) of a
// slot, L3[25][27] over trits (2,3,4), tail[27] over trits 125..127.
constexpr int kL2Entries = 9;
constexpr int kL3Entries = 27;
constexpr int kL3Base = kFullSlots * kL2Entries;             // 225
constexpr int kTailBase = kL3Base + kFullSlots * kL3Entries;  // 900
constexpr int kLutFloats = kTailBase + 27;                    // 927

// LUT23 split of a code byte p into its table digits: high = (p * 57) >> 9,
// equal to p / 9 for p <= 511, and low = p - 9 * high. V is unsigned short,
// or a vector of them (the kernels split two bytes per 16-bit-packed
// operation). For every byte value high <= 28 and low <= 8.
template <typename V>
__host__ __device__ __attribute__((always_inline)) inline V lut23_high(V p) {
    return (p * static_cast<unsigned short>(57)) >> static_cast<unsigned short>(9);
}
template <typename V>
__host__ __device__ __attribute__((always_inline)) inline V lut23_low(V p, V high) {
    return p - high * static_cast<unsigned short>(9);
}

// The other split of a code byte, into its three low and two high digits:
// high = (p * 19) >> 9, equal to p / 27 for every byte value, and low =
// p - 27 * high (0..26). For every byte value high <= 9.
template <typename V>
__host__ __device__ __attribute__((always_inline)) inline V split27_high(V p) {
    return (p * static_cast<unsigned short>(19)) >> static_cast<unsigned short>(9);
}
template <typename V>
__host__ __device__ __attribute__((always_inline)) inline V split27_low(V p, V high) {
    return p - high * static_cast<unsigned short>(27);
}

// Selector tables of the MFMA decoders. A weight with digit d is bytes
// (2d, 2d + 1) of the 8-byte table {-s, z, +s, 0} that v_perm_b32 selects
// from, so a dword of two weights' selectors turns into their fp16 pair with
// one v_perm_b32. A pair of consecutive code bytes (a, b) gives its ten
// weights as five pairs (digit i of a byte has weight 3^i):
//   (a0, a1) = T9a[a % 9]
//   (a2, a3) = T27aX[a / 9]
//   (a4, b0) = T27aY[a / 9] | T27bX[b % 27]
//   (b1, b2) = T27bY[b % 27]
//   (b3, b4) = T9b[b / 27]
// The tail byte t (three digits) reads as a b byte's low part: (t0 in the
// high half) = T27bX[t], (t1, t2) = T27bY[t]. Each table is at most 29 dwords, so a
// wave's lookups into one never conflict in the LDS banks. Indices of illegal
// bytes (a / 9 up to 28, b / 27 up to 9) stay inside their tables; their
// entries select bytes 6-7 of the table, a zero.
constexpr int kSelT9a = 0;     // 9 entries: l = a0 + 3 a1
constexpr int kSelT27aX = 9;   // 29 entries: h = a2 + 3 a3 + 9 a4
constexpr int kSelT27aY = 38;  // 29 entries, the same index: a4 in the low half
constexpr int kSelT27bX = 67;  // 27 entries: m = b0 + 3 b1 + 9 b2: b0 in the high half
constexpr int kSelT27bY = 94;  // 27 entries, the same index: (b1, b2)
constexpr int kSelT9b = 121;   // 10 entries: n = b3 + 3 b4
constexpr int kSelEntries = 131;

__host__ __device__ __attribute__((always_inline)) inline uint32_t selector_half(uint32_t d) {
    return (2u * d) | ((2u * d + 1u) << 8);
}
__host__ __device__ __attribute__((always_inline)) inline uint32_t selector_pair(uint32_t d_even, uint32_t d_odd) {
    return selector_half(d_even) | (selector_half(d_odd) << 16);
}

// Entry i of the concatenated selector tables.
__host__ __device__ inline uint32_t selector_entry(int i) {
    if (i < kSelT27aX) return selector_pair(i % 3, i / 3);
    if (i < kSelT27aY) {
        const int h = i - kSelT27aX;
        return selector_pair(h % 3, (h / 3) % 3);
    }
    if (i < kSelT27bX) return selector_half((i - kSelT27aY) / 9);
    if (i < kSelT27bY) return selector_half((i - kSelT27bX) % 3) << 16;
    if (i < kSelT9b) {
        const int m = i - kSelT27bY;
        return selector_pair((m / 3) % 3, m / 9);
    }
    const int n = i - kSelT9b;
    return selector_pair(n % 3, n / 3);
}

// Tail-table entry of a tail byte: the byte itself, clamped to the table.
__host__ __device__ __attribute__((always_inline)) inline uint32_t tail_entry(uint32_t p) {
    return p < kMaxTailByte ? p : kMaxTailByte;
}

// Product of the low 24 bits of a and b, low 32 bits of the result (one
// v_mul_u32_u24 on CDNA).
__host__ __device__ __attribute__((always_inline)) inline uint32_t mul24(uint32_t a, uint32_t b) {
    return (a & 0xffffffu) * (b & 0xffffffu);
}

// Digit carriers: t = p * 69043 approximates p / 243 in 24-bit fixed point
// and each step t = (t mod 2^24) * 3 leaves the next base-3 digit, most
// significant first, in bits 24-25 (and zeros above: t < 3 * 2^24). Exact for
// every code byte p <= 242; the tail byte (p <= 26) uses 9 * 69043 ~ 2^24 / 27.
constexpr uint32_t kByteDigitScale = 69043u;       // ~2^24 / 243
constexpr uint32_t kTailDigitScale = 9u * 69043u;  // ~2^24 / 27

// d[i] carries digit i (weight 3^i) of code byte p in bits 24-25.
__host__ __device__ __attribute__((always_inline)) inline void byte_digit_carriers(uint32_t p,
                                                                                   uint32_t (&d)[5]) {
    uint32_t t = mul24(p, kByteDigitScale);
#pragma unroll
    for (int i = 4; i >= 0; --i) {
        t = mul24(t, 3u);
        d[i] = t;
    }
}

// d[i] carries digit i (weight 3^i) of tail byte p in bits 24-25.
__host__ __device__ __attribute__((always_inline)) inline void tail_digit_carriers(uint32_t p,
                                                                                   uint32_t (&d)[3]) {
    uint32_t t = mul24(p, kTailDigitScale);
#pragma unroll
    for (int i = 2; i >= 0; --i) {
        t = mul24(t, 3u);
        d[i] = t;
    }
}

// The five base-3 digits of byte b, digit i in bits 2i..2i+1 (the gather's
// per-byte table). Every digit is in 0..2 for every byte value (a byte over
// 242 loses its multiple of 243), so the word is below 2^10 and three bytes'
// digits pack into 30 bits.
__host__ __device__ __attribute__((always_inline)) inline uint32_t byte_digits(uint32_t b) {
    uint32_t d = 0;
#pragma unroll
    for (int i = 0; i < 5; ++i) {
        const uint32_t q = b / 3u;
        d |= (b - 3u * q) << (2 * i);
        b = q;
    }
    return d;
}

}  // namespace tq1_bytes

#endif  // TERNEL_TQ1_BYTES_H
