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

    // The selector tables of the MFMA decoders.
    unsigned max_high27 = 0;
    for (unsigned p = 0; p < 256; ++p) {
        const unsigned short a = static_cast<unsigned short>(p);
        const unsigned short h9 = lut23_high(a), l9 = lut23_low(a, h9);
        const unsigned short h27 = split27_high(a), l27 = split27_low(a, h27);
        max_high27 = h27 > max_high27 ? h27 : max_high27;
        expect(h27 == p / 27 && l27 == p % 27, "split27 is p / 27, p % 27 for every byte value", p);
        expect(kSelT9a + l9 < kSelT27aX, "T9a index inside T9a", p);
        expect(kSelT27aX + h9 < kSelT27aY && kSelT27aY + h9 < kSelT27bX, "T27a index inside T27aX, T27aY", p);
        expect(kSelT27bX + l27 < kSelT27bY && kSelT27bY + l27 < kSelT9b, "T27b index inside T27bX, T27bY", p);
        expect(kSelT9b + h27 < kSelEntries, "T9b index inside T9b", p);
        const unsigned t = tail_entry(p);
        expect(kSelT27bX + t < kSelT27bY && kSelT27bY + t < kSelT9b, "tail index inside T27bX, T27bY", p);
    }
    for (unsigned a = 0; a < 256; ++a)
        for (unsigned b = 0; b < 256; ++b) {
            const u16x2 pair = {static_cast<unsigned short>(a), static_cast<unsigned short>(b)};
            const u16x2 high = split27_high(pair);
            const u16x2 low = split27_low(pair, high);
            expect(high[0] == a / 27 && high[1] == b / 27 && low[0] == a % 27 && low[1] == b % 27,
                   "packed split27 equals the per-byte split", a, b);
        }
    for (unsigned a = 0; a <= kMaxCodeByte; ++a)
        for (unsigned b = 0; b <= kMaxCodeByte; ++b) {
            const unsigned la = a % 9, ha = a / 9, lb = b % 27, hb = b / 27;
            const uint32_t got[5] = {selector_entry(kSelT9a + la), selector_entry(kSelT27aX + ha),
                                     selector_entry(kSelT27aY + ha) | selector_entry(kSelT27bX + lb),
                                     selector_entry(kSelT27bY + lb), selector_entry(kSelT9b + hb)};
            unsigned d[10];
            for (int i = 0; i < 5; ++i) {
                d[i] = digit(a, i);
                d[5 + i] = digit(b, i);
            }
            for (int q = 0; q < 5; ++q)
                expect(got[q] == selector_pair(d[2 * q], d[2 * q + 1]), "byte pair's selectors are its digits' pairs", a,
                       static_cast<int>(b * 8 + q));
        }
    for (unsigned p = 0; p <= kMaxCodeByte; ++p)
        for (unsigned t = 0; t <= kMaxTailByte; ++t) {
            // code byte 24's fifth digit with the tail's first; the tail's last two
            const uint32_t lead = selector_entry(kSelT27aY + p / 9) | selector_entry(kSelT27bX + tail_entry(t));
            const uint32_t rest = selector_entry(kSelT27bY + tail_entry(t));
            expect(lead == selector_pair(digit(p, 4), digit(t, 0)), "byte 24 and tail lead pair", p, t);
            expect(rest == selector_pair(digit(t, 1), digit(t, 2)), "tail rest pair", p, t);
        }
    for (int i = 0; i < kSelEntries; ++i)
        for (int k = 0; k < 4; ++k)
            expect(((selector_entry(i) >> (8 * k)) & 0xffu) <= 7, "selector bytes pick inside the 8-byte table", i, k);
    const int table_sizes[6] = {kSelT27aX - kSelT9a, kSelT27aY - kSelT27aX, kSelT27bX - kSelT27aY,
                                kSelT27bY - kSelT27bX, kSelT9b - kSelT27bY, kSelEntries - kSelT9b};
    for (int i = 0; i < 6; ++i) expect(table_sizes[i] <= 32, "each selector table within 32 banks", i);
    printf("selector tables: %d entries; split27 high <= %u; every byte pair (a, b) <= 242 gives its ten digits' "
           "selector pairs, byte 24 with every tail byte too; every index of all 256 byte values inside its table\n",
           kSelEntries, max_high27);

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
