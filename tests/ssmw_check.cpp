// Drives the SSMW checkpoint validator (ssmjs_amd/csrc/ssmw.cpp) with valid, truncated,
// oversized, corrupted and randomly mutated images; built with AddressSanitizer and
// UndefinedBehaviorSanitizer by tests/test_sanitizers.py. Every image must either validate or
// be rejected with a reason, reading nothing outside its bytes. Prints "ok <counts>" and exits
// 0, or prints the first failure and exits 1.
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <vector>

#include "ssmw.hpp"

namespace {

int fails = 0;
#define CHECK(c, ...)                                   \
    do {                                                \
        if (!(c)) {                                     \
            std::printf("FAIL line %d: ", __LINE__);     \
            std::printf(__VA_ARGS__);                   \
            std::printf("\n");                          \
            ++fails;                                    \
        }                                               \
    } while (0)

uint64_t rs = 0x9E3779B97F4A7C15ull;
uint64_t rnd() {
    rs ^= rs << 13;
    rs ^= rs >> 7;
    rs ^= rs << 17;
    return rs;
}

// Validate a copy in a buffer of exactly `n` bytes (so ASan sees any read past the image).
const char* check_copy(const std::vector<unsigned char>& img, size_t n, const ssmw::Expect& e,
                       ssmw::Header* h) {
    std::vector<unsigned char> buf(img.begin(), img.begin() + (long)std::min(n, img.size()));
    buf.resize(n, 0xAB);
    buf.shrink_to_fit();
    return ssmw::validate(n ? buf.data() : nullptr, n, e, h);
}

}  // namespace

int main() {
    const int32_t dims[9] = {16, 8, 3, 4, 4, 2, 2, 1, 1};
    const unsigned char types[3] = {1, 2, 1};
    const uint64_t nfloats = 1000;
    const ssmw::Expect e{{16, 8, 3, 4, 4, 2, 2, 1, 1}, types, nfloats};
    long n_valid = 0, n_rejected = 0;
    for (int f16 = 0; f16 < 2; ++f16) {
        const size_t hb = ssmw::header_bytes(3), pay = nfloats * (f16 ? 2 : 4);
        std::vector<unsigned char> img(hb + pay);
        ssmw::write_header(dims, 1e-5f, 256, 0, 1, types, nfloats, f16, img.data());
        std::vector<float> w(nfloats);
        for (uint64_t i = 0; i < nfloats; ++i) {
            w[i] = (float)((double)(rnd() >> 11) / 9007199254740992.0 - 0.5) * 4.f;
            if (f16) {
                const uint16_t v = ssmw::f2h(w[i]);
                std::memcpy(img.data() + hb + 2 * i, &v, 2);
                w[i] = ssmw::h2f(v);
            } else {
                std::memcpy(img.data() + hb + 4 * i, &w[i], 4);
            }
        }
        ssmw::Header h;
        CHECK(check_copy(img, img.size(), e, &h) == nullptr, "valid image rejected (f16 %d)", f16);
        ++n_valid;
        std::vector<float> back(nfloats);
        ssmw::decode_payload(img.data() + hb, h, back.data());
        CHECK(std::memcmp(back.data(), w.data(), nfloats * 4) == 0, "payload round trip (f16 %d)", f16);
        // every truncation, and images one and sixteen bytes too long
        for (size_t n = 0; n < img.size(); ++n) {
            CHECK(check_copy(img, n, e, nullptr) != nullptr, "truncated to %zu accepted", n);
            ++n_rejected;
        }
        for (size_t extra : {1, 16}) {
            CHECK(check_copy(img, img.size() + extra, e, nullptr) != nullptr, "+%zu accepted", extra);
            ++n_rejected;
        }
        // each header byte changed: fields the validator checks must reject it, the free ones
        // (eps, chunk, eos, mimo, reserved, padding) may not
        for (size_t i = 0; i < hb; ++i) {
            std::vector<unsigned char> bad = img;
            bad[i] ^= 0x5A;
            const bool checked = i < 60 || (i >= 80 && i < 83);
            const char* why = check_copy(bad, bad.size(), e, nullptr);
            if (checked) CHECK(why != nullptr, "header byte %zu changed, accepted", i);
            why ? ++n_rejected : ++n_valid;
        }
        // payload-size fields that would wrap header + payload around 2^64
        for (uint64_t p : {~0ull, ~0ull - hb + 1, (uint64_t)pay + (1ull << 63), 1ull << 63}) {
            std::vector<unsigned char> bad = img;
            std::memcpy(bad.data() + 16, &p, 8);
            CHECK(check_copy(bad, bad.size(), e, nullptr) != nullptr, "payload field %llu accepted",
                  (unsigned long long)p);
            ++n_rejected;
        }
        // random mutations: length and up to eight byte edits, anywhere
        for (int it = 0; it < 20000; ++it) {
            std::vector<unsigned char> bad = img;
            const int edits = (int)(rnd() % 9);
            for (int k = 0; k < edits; ++k) bad[rnd() % bad.size()] = (unsigned char)rnd();
            const size_t n = (rnd() % 4 == 0) ? (size_t)(rnd() % (img.size() + 32)) : bad.size();
            ssmw::Header hh;
            const char* why = check_copy(bad, n, e, &hh);
            if (!why) {
                // accepted: then it has the expected size, and decoding stays inside it
                CHECK(n == img.size(), "mutated image of %zu bytes accepted", n);
                std::vector<float> out(nfloats);
                ssmw::decode_payload(bad.data() + hh.header_bytes, hh, out.data());
                ++n_valid;
            } else {
                ++n_rejected;
            }
        }
    }
    // f16 codec: every half value survives h2f -> f2h (NaNs stay NaNs)
    for (uint32_t v = 0; v < 65536; ++v) {
        const float f = ssmw::h2f((uint16_t)v);
        const uint16_t b = ssmw::f2h(f);
        if (std::isnan(f)) CHECK(std::isnan(ssmw::h2f(b)), "NaN %04x", v);
        else CHECK(b == v, "half %04x -> %04x", v, b);
    }
    // f32 -> f16 rounding at the edges: largest finite, overflow, smallest subnormal, ties
    CHECK(ssmw::f2h(65504.f) == 0x7bff, "max half");
    CHECK(ssmw::f2h(65520.f) == 0x7c00, "overflow to inf");
    CHECK(ssmw::f2h(std::ldexp(1.f, -24)) == 0x0001, "smallest subnormal");
    CHECK(ssmw::f2h(1.f + std::ldexp(1.f, -11)) == 0x3c00, "tie to even (down)");
    CHECK(ssmw::f2h(1.f + 3 * std::ldexp(1.f, -11)) == 0x3c02, "tie to even (up)");
    if (fails) return 1;
    std::printf("ok valid %ld rejected %ld\n", n_valid, n_rejected);
    return 0;
}
