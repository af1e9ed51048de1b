// Host-side check of address_from_words (csrc/kernels/common.hpp), the
// widening that every write-through store descriptor (WtOut) applies to the
// two words of its base after __builtin_amdgcn_readfirstlane. Built with
// hipcc for the host only by tests/test_descriptor_base.py.
//
// For each (low word, high word) pair the address must be hi:lo exactly. The
// widening that faulted on the GPU (each int word cast straight to 64 bits)
// is kept here as `signed_widening` to show that the cases below tell the two
// apart: it must disagree wherever the low word has bit 31 set.
#include <cstdio>
#include <cstdint>

#include "kernels/common.hpp"

static uint64_t signed_widening(int lo, int hi) { return ((uint64_t)(int64_t)hi << 32) | (uint64_t)(int64_t)lo; }

static_assert(dhx::address_from_words((int)0x80000000u, 0) == 0x80000000ull, "bit 31 of the low word");
static_assert(dhx::address_from_words(-1, 0x7f) == 0x7fffffffffull, "all-ones low word");

int main() {
    const uint32_t lows[] = {0u, 1u, 0x7fffffffu, 0x80000000u, 0x80000100u, 0xfffff000u, 0xffffffffu};
    const uint32_t highs[] = {0u, 1u, 0x7fu, 0x7fffu, 0x12345u, 0x7fffffffu, 0xffffffffu};
    int failures = 0, told_apart = 0, bit31 = 0;
    for (uint32_t lo : lows)
        for (uint32_t hi : highs) {
            const uint64_t want = ((uint64_t)hi << 32) | lo;
            // The words go through int exactly as readfirstlane returns them.
            const uint64_t got = dhx::address_from_words((int)lo, (int)hi);
            if (got != want) {
                std::printf("FAIL lo %08x hi %08x: %016llx, want %016llx\n", lo, hi, (unsigned long long)got,
                            (unsigned long long)want);
                ++failures;
            }
            const bool old_wrong = signed_widening((int)lo, (int)hi) != want;
            if (lo & 0x80000000u) {
                ++bit31;
                told_apart += old_wrong;
            } else if (old_wrong) {
                std::printf("the signed widening disagrees without bit 31: lo %08x hi %08x\n", lo, hi);
                ++failures;
            }
        }
    // Every bit-31 case must expose the old widening, or this test would not
    // have caught it (with hi = 0xffffffff the sign extension is invisible).
    const int expected_apart = bit31 - 4;  // four bit-31 lows x the one all-ones high word
    if (told_apart != expected_apart) {
        std::printf("the cases expose the signed widening %d times, want %d\n", told_apart, expected_apart);
        ++failures;
    }
    std::printf("%d cases, %d with bit 31 of the low word, %d expose the signed widening, %d failures\n",
                (int)(sizeof(lows) / sizeof(lows[0]) * sizeof(highs) / sizeof(highs[0])), bit31, told_apart,
                failures);
    return failures == 0 ? 0 : 1;
}
