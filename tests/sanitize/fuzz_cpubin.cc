// fuzz_cpubin.cc — the .cpu.bin reader (tabinfer_amd/csrc/ti_cpubin.hip, host C++) under
// AddressSanitizer and UndefinedBehaviorSanitizer, CPU only:
//   fuzz_cpubin <iterations> <seed>
// First the corrupted-container cases of native/crates/n2-core/src/binfmt.rs:430-482 (a
// misaligned header reads; codesLen != N*K/4 and an overrunning range are refused with
// the reference's words). Then seeded mutations of a valid container — bytes flipped or
// replaced by JSON punctuation in the header, numbers swapped for extreme values, the
// header length field rewritten, the file cut short — each parsed, and every accessor run
// on whatever parses: every tensor's byte ranges are read in full and embedding rows are
// fetched at in-range, edge and absurd indices. The first failure ends the run with exit
// status 1 (a sanitizer report aborts it before that).
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <string>
#include <vector>
#include "ti.h"

static uint64_t g_rng = 0x9E3779B97F4A7C15ull;
static uint64_t next_u64() {   // xorshift64*
    g_rng ^= g_rng >> 12;
    g_rng ^= g_rng << 25;
    g_rng ^= g_rng >> 27;
    return g_rng * 2685821657736338717ull;
}
static uint64_t below(uint64_t n) { return n ? next_u64() % n : 0; }

static std::vector<uint8_t> container(const std::string& header, size_t blob_len, uint8_t fill) {
    std::vector<uint8_t> f(4 + header.size() + blob_len, fill);
    const uint32_t hl = (uint32_t)header.size();
    memcpy(f.data(), &hl, 4);
    memcpy(f.data() + 4, header.data(), header.size());
    return f;
}

static int fail(const char* what, const char* detail) {
    fprintf(stderr, "FAIL: %s: %s\n", what, detail ? detail : "");
    return 1;
}

// every accessor on a parsed container; returns nonzero on an inconsistent answer
static volatile uint64_t g_sink = 0;
static int exercise(const ti_cpubin* c) {
    int G = 0, n = 0;
    size_t blob = 0;
    if (ti_cpubin_summary(c, &G, &n, &blob)) return fail("summary", ti_last_error());
    if (G != 64) return fail("summary", "G != 64 accepted");
    for (int i = 0; i < n; i++) {
        const char* name = nullptr;
        if (ti_cpubin_name(c, i, &name) || !name) return fail("name", ti_last_error());
        ti_cpubin_tensor_info t;
        if (ti_cpubin_tensor(c, name, &t)) continue;   // a refused view (misaligned f32) is fine
        // read every byte the view claims: an overrun is a sanitizer report
        const uint8_t* d = static_cast<const uint8_t*>(t.data);
        uint64_t s = 0;
        for (size_t k = 0; k < t.data_bytes; k++) s += d[k];
        if (t.scales) {
            const uint8_t* q = static_cast<const uint8_t*>(t.scales);
            for (size_t k = 0; k < t.scale_bytes; k++) s += q[k];
        }
        g_sink = g_sink + s;
        if (t.kind == TI_CPUBIN_TERN && (t.K % 64 != 0 || (size_t)(t.N * (t.K / 4)) != t.data_bytes))
            return fail("tensor", "a ternary view that breaks codesLen = N*K/4");
        if (t.kind == TI_CPUBIN_EMBED_F16 && t.ndim > 0) {
            const long long dim = t.shape[t.ndim - 1];
            if (dim <= 0 || dim > (1 << 16)) continue;
            std::vector<float> row((size_t)dim);
            const long long rows = (long long)(t.data_bytes / (2 * (size_t)dim));
            const long long probe[] = {0, rows - 1, rows, rows + 1, -1, (long long)1 << 40, 0x7fffffffffffffffll / dim,
                                       0x7fffffffffffffffll};
            for (long long r : probe) {
                const int rc = ti_cpubin_embed_row(c, name, r, row.data(), (int)dim);
                if (r >= 0 && r < rows && rc) return fail("embed_row", ti_last_error());
                if ((r < 0 || r >= rows) && !rc) return fail("embed_row", "an out-of-range row was read");
            }
            if (ti_cpubin_embed_row(c, name, 0, row.data(), (int)dim + 1) == 0) return fail("embed_row", "wrong dim accepted");
        }
    }
    const char* none = nullptr;
    if (ti_cpubin_name(c, n, &none) == 0 || ti_cpubin_name(c, -1, &none) == 0) return fail("name", "an index past the end");
    return 0;
}

static int known_cases() {
    // misaligned header (its length not a multiple of 4): the blob still reads
    {
        const std::string h = "{\"G\":64,\"tensors\":{\"lm_head.weight\":{\"kind\":\"tern\",\"N\":2,\"K\":64,\"codesOff\":0,"
                              "\"codesLen\":32,\"scalesOff\":32,\"scalesLen\":8}}} ";
        std::string hh = h;
        while (hh.size() % 4 == 0) hh += " ";
        std::vector<uint8_t> f = container(hh, 48, 0);
        const float sc[2] = {1.5f, 2.5f};
        memcpy(f.data() + 4 + hh.size() + 32, sc, 8);
        ti_cpubin* c = nullptr;
        if (ti_cpubin_parse(f.data(), f.size(), &c)) return fail("misaligned header", ti_last_error());
        ti_cpubin_tensor_info t;
        if (ti_cpubin_tensor(c, "lm_head.weight", &t) || t.N != 2 || t.K != 64 || t.data_bytes != 32 ||
            ((uintptr_t)t.scales & 3) || static_cast<const float*>(t.scales)[0] != 1.5f ||
            static_cast<const float*>(t.scales)[1] != 2.5f)
            return fail("misaligned header", "wrong view");
        if (exercise(c)) return 1;
        ti_cpubin_close(c);
    }
    // codesLen deliberately wrong for N*K/4
    {
        const std::string h = "{\"G\":64,\"tensors\":{\"w\":{\"kind\":\"tern\",\"N\":2,\"K\":64,\"codesOff\":0,\"codesLen\":99,"
                              "\"scalesOff\":32,\"scalesLen\":8}}}";
        std::vector<uint8_t> f = container(h, 128, 0);
        ti_cpubin* c = nullptr;
        if (ti_cpubin_parse(f.data(), f.size(), &c) == 0 || !strstr(ti_last_error(), "codesLen"))
            return fail("shape mismatch", ti_last_error());
    }
    // a range past the blob
    {
        const std::string h = "{\"G\":64,\"tensors\":{\"w\":{\"kind\":\"f32\",\"shape\":[4],\"off\":0,\"len\":4096}}}";
        std::vector<uint8_t> f = container(h, 16, 0);
        ti_cpubin* c = nullptr;
        if (ti_cpubin_parse(f.data(), f.size(), &c) == 0 || !strstr(ti_last_error(), "overruns"))
            return fail("overrunning range", ti_last_error());
    }
    return 0;
}

// a valid container holding one tensor of each kind
static std::vector<uint8_t> seed_container(size_t* header_len) {
    const std::string h =
        "{\"G\":64,\"tensors\":{"
        "\"lm_head.weight\":{\"kind\":\"tern\",\"N\":4,\"K\":128,\"codesOff\":0,\"codesLen\":128,\"scalesOff\":128,\"scalesLen\":32},"
        "\"model.embed_tokens.weight\":{\"kind\":\"embed_f16\",\"shape\":[6,8],\"off\":160,\"len\":96},"
        "\"model.norm.weight\":{\"kind\":\"f32\",\"shape\":[8],\"off\":256,\"len\":32},"
        "\"x\\u0041\\n\":{\"kind\":\"f32\",\"shape\":[2,2],\"off\":288,\"len\":16}}}";
    *header_len = h.size();
    std::vector<uint8_t> f = container(h, 320, 0);
    for (size_t i = 4 + h.size(); i < f.size(); i++) f[i] = (uint8_t)(i * 131u);
    return f;
}

static const char* const EXTREMES[] = {"18446744073709551615", "18446744073709551616", "9223372036854775807",
                                       "-9223372036854775808", "-1", "0", "1e308", "-1e308", "1.5", "4294967296",
                                       "99999999999999999999999", "NaN", "\"64\"", "null", "[]", "{}", "true"};

int main(int argc, char** argv) {
    const long iters = argc > 1 ? atol(argv[1]) : 20000;
    g_rng ^= (argc > 2 ? strtoull(argv[2], nullptr, 10) : 1) * 0xD1B54A32D192ED03ull;
    if (known_cases()) return 1;
    size_t hl0 = 0;
    const std::vector<uint8_t> seed = seed_container(&hl0);
    {
        ti_cpubin* c = nullptr;
        if (ti_cpubin_parse(seed.data(), seed.size(), &c)) return fail("seed", ti_last_error());
        if (exercise(c)) return 1;
        ti_cpubin_close(c);
    }
    long parsed = 0;
    for (long it = 0; it < iters; it++) {
        std::vector<uint8_t> f = seed;
        size_t hl = hl0;
        const int nmut = 1 + (int)below(4);
        for (int m = 0; m < nmut; m++) {
            // the header bytes still present (a cut can leave fewer than its length field says)
            hl = f.size() >= 4 ? (hl < f.size() - 4 ? hl : f.size() - 4) : 0;
            switch (below(7)) {
                case 0: if (hl) f[4 + below(hl)] ^= (uint8_t)(1u << below(8)); break;
                case 1: if (hl) f[4 + below(hl)] = (uint8_t)"{}[]\":,-+.eE0123456789\\u \x00\xff"[below(27)]; break;
                case 2: {   // a number in the header replaced by an extreme literal
                    if (!hl) break;
                    std::string h(f.begin() + 4, f.begin() + 4 + hl);
                    size_t p = h.find_first_of("0123456789", below(h.size()));
                    if (p == std::string::npos) break;
                    size_t q = h.find_first_not_of("0123456789", p);
                    if (q == std::string::npos) q = h.size();
                    h.replace(p, q - p, EXTREMES[below(sizeof EXTREMES / sizeof EXTREMES[0])]);
                    std::vector<uint8_t> g(4 + h.size() + (f.size() - 4 - hl));
                    const uint32_t nh = (uint32_t)h.size();
                    memcpy(g.data(), &nh, 4);
                    memcpy(g.data() + 4, h.data(), h.size());
                    memcpy(g.data() + 4 + h.size(), f.data() + 4 + hl, f.size() - 4 - hl);
                    f.swap(g);
                    hl = h.size();
                    break;
                }
                case 3: {   // the header length field rewritten
                    const uint32_t v = below(3) == 0 ? (uint32_t)next_u64() : (uint32_t)(hl + below(64) - 32);
                    memcpy(f.data(), &v, 4);
                    break;
                }
                case 4: f.resize(below(f.size() + 1)); break;                      // cut short
                case 5: if (hl > 2) { f.erase(f.begin() + 4 + (long)below(hl)); } break;   // a byte dropped, length kept
                default: {   // a byte inserted, length kept
                    const size_t at = 4 + below(hl + 1);
                    if (at <= f.size()) f.insert(f.begin() + (long)at, (uint8_t)below(256));
                }
            }
            if (f.size() < 4) break;
        }
        ti_cpubin* c = nullptr;
        const int rc = ti_cpubin_parse(f.data(), f.size(), &c);
        if (rc == 0) {
            parsed++;
            if (!c) return fail("parse", "OK without a container");
            if (exercise(c)) {
                fprintf(stderr, "at iteration %ld\n", it);
                return 1;
            }
            ti_cpubin_close(c);
        } else if (c) {
            return fail("parse", "an error left a container behind");
        } else if (!ti_last_error()[0]) {
            return fail("parse", "an error without a message");
        }
    }
    printf("ok %ld iterations, %ld parsed, sink %llu\n", iters, parsed, (unsigned long long)(g_sink & 1));
    return 0;
}
