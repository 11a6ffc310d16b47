// Exhaustive host-side check of the byte arithmetic the TQ1_G128 kernels share
// through ternel_amd/csrc/tq1_bytes.h, over every byte value 0..255 (legal or
// not): table entries stay inside their group's LUT23 table, digit carriers
// hold digits in 0..2 with nothing above them, the gather's digit table packs
// without overlap, and legal bytes give their exact base-3 digits (compared
// with plain division). Built and run by tests/test_byte_bounds.py with a host
// compiler (__host__ / __device__ defined empty). Prints one line per property
// group, the first 20 violations, and exits nonzero if there was any.
#include <stdint.h>
#include <stdio.h>

#include "tq1_bytes.h"

using namespace tq1_bytes;

namespace {

int failures = 0;

void expect(bool ok, const char *what, unsigned p, int extra = -1) {
    if (ok) return;
    if (failures++ < 20) printf("FAIL %s: byte %u (%d)\n", what, p, extra);
}

unsigned digit(unsigned p, int i) {
    for (int k = 0; k < i; ++k) p /= 3;
    return p % 3;
}

typedef unsigned short u16x2 __attribute__((vector_size(4)));

}  // namespace

int main() {
    // LUT23 split, one byte at a time and two per 16-bit-packed operation.
    unsigned max_high = 0, max_low = 0;
    for (unsigned p = 0; p < 256; ++p) {
        const unsigned short high = lut23_high(static_cast<unsigned short>(p));
        const unsigned short low = lut23_low(static_cast<unsigned short>(p), high);
        max_high = high > max_high ? high : max_high;
        max_low = low > max_low ? low : max_low;
        expect(low <= 8, "low digit <= 8", p, low);
        if (p <= kMaxCodeByte) {
            expect(high == p / 9 && low == p % 9, "legal byte splits into p / 9, p % 9", p);
            expect(high < static_cast<unsigned>(kL3Entries), "legal high digit inside its L3 slot", p, high);
        }
        for (int s = 0; s < kFullSlots; ++s) {
            const int l2 = s * kL2Entries + low;
            const int l3 = kL3Base + s * kL3Entries + high;
            expect(l2 >= 0 && l2 < kL3Base, "L2 entry inside the L2 tables", p, s);
            expect(l3 >= kL3Base && l3 < kLutFloats, "L3 entry inside the group's table", p, s);
        }
        const int tail = kTailBase + static_cast<int>(tail_entry(p));
        expect(tail >= kTailBase && tail < kLutFloats, "tail entry inside the tail table", p);
        if (p <= kMaxTailByte) expect(tail_entry(p) == p, "legal tail byte is its own entry", p);
    }
    for (unsigned a = 0; a < 256; ++a)
        for (unsigned b = 0; b < 256; ++b) {
            const u16x2 pair = {static_cast<unsigned short>(a), static_cast<unsigned short>(b)};
            const u16x2 high = lut23_high(pair);
            const u16x2 low = lut23_low(pair, high);
            const unsigned short ha = lut23_high(static_cast<unsigned short>(a));
            const unsigned short hb = lut23_high(static_cast<unsigned short>(b));
            expect(high[0] == ha && high[1] == hb, "packed split equals the per-byte split (high)", a, b);
            expect(low[0] == lut23_low(static_cast<unsigned short>(a), ha) &&
                       low[1] == lut23_low(static_cast<unsigned short>(b), hb),
                   "packed split equals the per-byte split (low)", a, b);
        }
    printf("lut23 split: 256 bytes, 65536 packed pairs; high <= %u, low <= %u; every L2/L3/tail entry of all %d "
           "slots inside the %d-entry group table\n",
           max_high, max_low, kFullSlots, kLutFloats);

    // Digit carriers of the MFMA decoders.
    for (unsigned p = 0; p < 256; ++p) {
        uint32_t d[5], t[3];
        byte_digit_carriers(p, d);
        tail_digit_carriers(p, t);
        for (int i = 0; i < 5; ++i) {
            expect((d[i] >> 26) == 0 && (d[i] >> 24) <= 2, "code carrier holds a digit in 0..2", p, i);
            if (p <= kMaxCodeByte) expect((d[i] >> 24) == digit(p, i), "legal code byte digit exact", p, i);
        }
        for (int i = 0; i < 3; ++i) {
            expect((t[i] >> 26) == 0 && (t[i] >> 24) <= 2, "tail carrier holds a digit in 0..2", p, i);
            if (p <= kMaxTailByte) expect((t[i] >> 24) == digit(p, i), "legal tail byte digit exact", p, i);
        }
    }
    printf("digit carriers: 256 code and 256 tail bytes; every carrier's top byte is a digit in 0..2 (a v_perm_b32 "
           "selector pair 2d, 2d+1 <= 5 picks a scale-table byte); legal bytes exact\n");

    // The gather's per-byte digit table.
    for (unsigned b = 0; b < 256; ++b) {
        const uint32_t d = byte_digits(b);
        expect(d < (1u << 10), "digit word below 2^10", b);
        unsigned value = 0, weight = 1;
        for (int i = 0; i < 5; ++i, weight *= 3) {
            expect(((d >> (2 * i)) & 3u) <= 2, "gather digit in 0..2", b, i);
            value += ((d >> (2 * i)) & 3u) * weight;
        }
        expect(value == b % 243, "digit word is the byte modulo 243", b);
        if (b <= kMaxCodeByte)
            for (int i = 0; i < 5; ++i) expect(((d >> (2 * i)) & 3u) == digit(b, i), "legal byte digits exact", b, i);
    }
    printf("gather digit table: 256 entries, digits in 0..2, below 2^10 (three bytes pack into 30 bits); legal bytes "
           "exact\n");

    if (failures) {
        printf("%d violations\n", failures);
        return 1;
    }
    printf("ok\n");
    return 0;
}
