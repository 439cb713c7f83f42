// Invariants of the split-KV attention plans of kudacuda_amd/csrc/kc_kernels.h,
// checked exhaustively on the host for every kv_len up to the largest
// standalone cache (65536 tokens):
//   * the round path (32-token units; caps 1..8, 32, 256) and the
//     matrix-core tactic (64- and 128-token units, cap 128);
//   * splits are whole units, there are at most `cap` of them, every token
//     lies in exactly one split (the last one non-empty), and no smaller
//     whole-unit size keeps the count within the cap;
//   * the count never exceeds min(cap, units of any larger capacity) -- the
//     grid bound the launchers size for device-side lengths.
// The matrix-core tactic's sums are not restated by the oracle, so this is
// where its partition of the tokens is pinned.
#include <cstdint>
#include <cstdio>

#include "../../kudacuda_amd/csrc/kc_kernels.h"

namespace {

int failures = 0;

void expect(bool ok, const char* what, int64_t L, int64_t unit, int64_t cap) {
    if (!ok && failures++ < 20) {
        std::printf("FAIL %s: L=%lld unit=%lld cap=%lld\n", what, static_cast<long long>(L),
                    static_cast<long long>(unit), static_cast<long long>(cap));
    }
}

template <typename Tokens, typename Count>
void check(int64_t unit, int64_t cap, Tokens tokens, Count count) {
    const int64_t max_len = 65536;
    for (int64_t L = 1; L <= max_len; ++L) {
        const int64_t C = tokens(L, cap);
        const int64_t n = count(L, cap);
        expect(C > 0 && C % unit == 0, "split is whole units", L, unit, cap);
        expect(n >= 1 && n <= cap, "count within the cap", L, unit, cap);
        expect(n == (L + C - 1) / C, "count covers L", L, unit, cap);
        expect((n - 1) * C < L && n * C >= L, "last split non-empty", L, unit, cap);
        if (C > unit) {
            const int64_t smaller = C - unit;
            expect((L + smaller - 1) / smaller > cap, "fewest units per split", L, unit, cap);
        }
        const int64_t units = (L + unit - 1) / unit;
        expect(n <= (units < cap ? units : cap), "grid bound for any capacity >= L", L, unit, cap);
    }
}

}  // namespace

int main() {
    for (int64_t cap : {1, 2, 3, 4, 5, 6, 7, 8, 32, 256}) {
        check(kc::kGqaRoundTokens, cap, [](int64_t L, int64_t c) { return kc::gqa_split_tokens(L, c); },
              [](int64_t L, int64_t c) { return kc::gqa_split_count(L, c); });
    }
    for (int64_t unit : {64, 128}) {
        check(unit, kc::kGqaMfmaSplitCap,
              [unit](int64_t L, int64_t c) { return kc::gqa_mfma_split_tokens(L, c, unit); },
              [unit](int64_t L, int64_t c) { return kc::gqa_mfma_split_count(L, c, unit); });
    }
    // the 2-wave blocks are chosen while one 64-token unit per split fits the cap
    for (int64_t L = 8192; L <= 8192 + 64; ++L) {
        const bool two = L <= 64 * kc::kGqaMfmaSplitCap;
        expect(!two || kc::gqa_mfma_split_tokens(L, kc::kGqaMfmaSplitCap, 64) == 64, "one unit per split", L, 64,
               kc::kGqaMfmaSplitCap);
    }
    if (failures != 0) {
        std::printf("%d failures\n", failures);
        return 1;
    }
    std::printf("split plan ok\n");
    return 0;
}
