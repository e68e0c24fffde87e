// host_checks.cpp — TEST INFRASTRUCTURE: a native driver for the host side, built by
// tests/test_native_host.py with AddressSanitizer and UndefinedBehaviorSanitizer (g++/gcc,
// CPU only). It restates the mix_decode known answers (engine/mod.rs:663-707) against the C++
// mirror's mix_decode, and runs the host C-ABI helpers (bfi_host.cpp) and the C oracle
// (oracle/bfi_oracle.c) over seeded random inputs, checking the helpers against the oracle
// where both exist. Prints "ok" and exits 0 when every check holds.
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>
#include <vector>

#include "../../builderforce-inference_amd/host/bfi_host.hpp"
#include "../../oracle/bfi_oracle.h"

static int g_fail = 0;
#define CHECK(c)                                                              \
    do {                                                                      \
        if (!(c)) {                                                           \
            std::fprintf(stderr, "check failed at line %d: %s\n", __LINE__, #c); \
            g_fail++;                                                         \
        }                                                                     \
    } while (0)

static uint64_t g_seed = 0x1234567887654321ull;
static uint64_t rnd() {  // splitmix64 (test inputs only)
    uint64_t z = (g_seed += 0x9E3779B97F4A7C15ull);
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}
static uint32_t rint_(uint32_t n) { return (uint32_t)(rnd() % n); }
static float rflt() { return (float)((rnd() >> 40) * (1.0 / 16777216.0)); }

// engine/mod.rs:663-690 mix_decode_four_streams_share_steps
static void mix_decode_four_streams_share_steps() {
    struct S {
        size_t left;
        uint64_t steps;
    };
    std::vector<S> seqs = {{3, 0}, {3, 0}, {2, 0}, {4, 0}};
    size_t sum = 0;
    for (auto& s : seqs) sum += s.left;
    const uint64_t steps = bfi::mix_decode(seqs, [](const S& s) { return s.left > 0; },
                                           [](S& s) {
                                               s.left -= 1;
                                               s.steps += 1;
                                           });
    CHECK(steps == 4);  // shared steps = max length, not sum
    CHECK(steps < sum);
    for (auto& s : seqs) CHECK(s.left == 0);
    CHECK(seqs[0].steps == 3);
    CHECK(seqs[3].steps == 4);
}

// engine/mod.rs:692-707 mix_decode_four_equal_streams_beats_serial
static void mix_decode_four_equal_streams_beats_serial() {
    struct S {
        size_t left;
    };
    std::vector<S> seqs(4, S{5});
    const size_t sum = 20;
    const uint64_t steps =
        bfi::mix_decode(seqs, [](const S& s) { return s.left > 0; }, [](S& s) { s.left -= 1; });
    CHECK(steps == 5);
    CHECK(steps < sum);
}

// mix_decode with nothing live takes no step (the all-done check comes first).
static void mix_decode_nothing_live() {
    std::vector<int> seqs = {0, 0};
    CHECK(bfi::mix_decode(seqs, [](const int& s) { return s > 0; }, [](int& s) { s--; }) == 0);
}

static void rng_and_seed() {
    for (int t = 0; t < 2000; t++) {
        uint64_t a = rnd() >> (rint_(4) * 16), b = a;  // (includes 0: the fixed replacement)
        if (t == 0) a = b = 0;
        for (int k = 0; k < 4; k++) {
            CHECK(bfi_rng_next_u64(&a) == orc_rng_next(&b));
            const float x = bfi_rng_f32(&a), y = orc_rng_f32(&b);
            CHECK(std::memcmp(&x, &y, 4) == 0);
        }
        const uint64_t s = rnd(), n = rnd() % 5000;
        CHECK(bfi_slot_rng_seed(s, n) == orc_slot_rng_seed(s, n));
    }
}

static void drafts() {
    std::vector<uint32_t> ctx, o1(16), o2(16);
    for (int t = 0; t < 3000; t++) {
        const size_t len = rint_(40);
        ctx.resize(len);
        for (auto& c : ctx) c = rint_(4);
        const size_t k = rint_(9), nmax = rint_(5), nmin = rint_(4);
        const size_t a = bfi_draft(ctx.data(), len, k, nmax, nmin, o1.data());
        const size_t b = orc_draft(ctx.data(), len, k, nmax, nmin, o2.data());
        CHECK(a == b);
        CHECK(std::memcmp(o1.data(), o2.data(), a * 4) == 0);
    }
}

static void id_unions() {
    // random grammars over pieces that exercise the parser: keywords, digits, separators and
    // multi-byte White_Space / non-whitespace code points, inserted at code point boundaries
    // (the reference's grammar is a Rust String: valid UTF-8)
    static const char* P[] = {"root", "::=", "id(", ")", "|", " ", "\t", "\n", "\xc2\xa0", "\xe3\x80\x80",
                              "\xe2\x80\xa8", "\xe2\x80\x8b", "\xef\xbb\xbf", "\xc2\x85", "+", "7", "42",
                              "4294967295", "4294967296", "x", "\""};
    const int NP = (int)(sizeof(P) / sizeof(P[0]));
    std::vector<uint32_t> m1(3), m2(3);
    for (int t = 0; t < 20000; t++) {
        std::string g;
        if (rint_(2)) g = "root ::= id(5)";
        const int n = (int)rint_(12);
        for (int i = 0; i < n; i++) {
            size_t at = rint_((uint32_t)g.size() + 1);
            while (at > 0 && at < g.size() && ((uint8_t)g[at] & 0xC0u) == 0x80u) at--;
            g.insert(at, P[rint_((uint32_t)NP)]);
        }
        std::fill(m1.begin(), m1.end(), 0xA5A5A5A5u);
        std::fill(m2.begin(), m2.end(), 0xA5A5A5A5u);
        const int a = bfi_parse_id_union(g.c_str(), 70, m1.data());
        const int b = orc_parse_id_union(g.c_str(), 70, m2.data());
        CHECK(a == b);
        if (a != b) std::fprintf(stderr, "  grammar [%s]: library %d oracle %d\n", g.c_str(), a, b);
        if (a && b) CHECK(m1 == m2);
    }
}

static void replays() {
    for (int t = 0; t < 5000; t++) {
        const size_t n = rint_(7);
        std::vector<uint32_t> d(n), out(n + 1);
        std::vector<uint8_t> stops(n);
        for (auto& x : d) x = rint_(5);
        for (auto& x : stops) x = rint_(4) == 0;
        uint64_t st = rnd();
        size_t np = 0, acc = 0;
        int done = 0;
        int64_t pend = 0;
        const int rc = bfi_spec_replay(d.data(), rint_(2) ? stops.data() : nullptr, n, (int32_t)rint_((uint32_t)n + 1),
                                       rint_(5), rint_(2) ? -1 : (int64_t)rint_(5), 1 + rint_(6), rint_(12), &st,
                                       out.data(), &np, &acc, &done, &pend);
        CHECK(rc == 0);
        CHECK(np <= n && acc == np);
        CHECK(!done || pend == -1);
    }
}

// The oracle's target / sample / verify over small random rows (sanitizer coverage of the
// checker itself; its values are pinned by the Python tests).
static void oracle_rows() {
    for (int t = 0; t < 3000; t++) {
        const size_t V = 1 + rint_(40);
        std::vector<float> x(V * 3);
        for (auto& v : x) v = (rflt() - 0.5f) * 20.0f;
        if (rint_(5) == 0) x[rint_((uint32_t)V)] = -INFINITY;
        std::vector<uint32_t> prev(rint_(8));
        for (auto& p : prev) p = rint_((uint32_t)V + 2);
        bfi_smp_row_params p{};
        p.temperature = rint_(4) == 0 ? 0.0f : 0.1f + 2.0f * rflt();
        p.top_k = (int32_t)rint_(6) - 1;
        p.top_p = rint_(3) == 0 ? 1.0f : rflt();
        p.min_p = rint_(3) == 0 ? 0.0f : rflt() * 1.2f;
        p.repeat_penalty = rint_(2) ? 1.0f : 0.5f + rflt();
        p.presence_penalty = rint_(2) ? 0.0f : rflt();
        p.frequency_penalty = rint_(2) ? 0.0f : rflt();
        std::vector<uint32_t> mask((V + 31) / 32, 0xFFFFFFFFu);
        if (rint_(3) == 0)
            for (auto& w : mask) w = (uint32_t)rnd();
        const uint32_t* mk = rint_(2) ? mask.data() : nullptr;
        std::vector<uint32_t> ids(V);
        std::vector<float> w(V), s(V);
        orc_target_info info;
        (void)orc_target(x.data(), V, prev.data(), prev.size(), &p, mk, ids.data(), w.data(), s.data(), &info);
        const uint32_t tok = orc_sample(x.data(), V, prev.data(), prev.size(), &p, mk, rflt());
        CHECK(tok < V);
        if (info.kind == 1 && info.len > 0) {
            uint32_t rej = 0;
            (void)orc_judge(info.kind, info.token, ids.data(), w.data(), (size_t)info.len, rint_((uint32_t)V), rflt(),
                            rflt(), &rej);
        }
        const uint32_t dr[2] = {rint_((uint32_t)V), rint_((uint32_t)V)};
        const float up[4] = {rflt(), rflt(), rflt(), rflt()};
        int32_t accd = -1;
        uint32_t nxt = 0;
        orc_verify_seq(x.data(), 0, (int64_t)V, (int64_t)V, &p, prev.data(), prev.size(), dr, 2, nullptr, 0, up, rflt(),
                       &accd, &nxt);
        CHECK(accd >= 0 && accd <= 2 && nxt < V);
    }
}

int main() {
    mix_decode_four_streams_share_steps();
    mix_decode_four_equal_streams_beats_serial();
    mix_decode_nothing_live();
    rng_and_seed();
    drafts();
    id_unions();
    replays();
    oracle_rows();
    if (g_fail) {
        std::fprintf(stderr, "%d checks failed\n", g_fail);
        return 1;
    }
    std::printf("ok\n");
    return 0;
}
