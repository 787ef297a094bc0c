// SSMW checkpoint images: validation, header and f16 codec (host code only).
#include "ssmw.hpp"

#include <cmath>
#include <cstring>

namespace ssmw {

const char* validate(const void* buf, size_t bytes, const Expect& e, Header* out) {
    const unsigned char* p = (const unsigned char*)buf;
    if (!p || bytes < 80 || std::memcmp(p, "SSMW", 4) != 0) return "bad magic";
    Header h;
    std::memcpy(&h.version, p + 4, 4);
    std::memcpy(&h.dtype, p + 8, 4);
    std::memcpy(&h.header_bytes, p + 12, 4);
    std::memcpy(&h.payload, p + 16, 8);
    std::memcpy(h.dims, p + 24, 36);
    std::memcpy(&h.eps, p + 60, 4);
    std::memcpy(&h.chunk, p + 64, 4);
    std::memcpy(&h.eos, p + 68, 4);
    std::memcpy(&h.mimo, p + 72, 4);
    if (h.version != kVersion) return "unsupported version";
    if (h.dtype > 1) return "unsupported dtype";
    const int nl = e.dims[2];
    if (h.dims[2] != nl || h.header_bytes != header_bytes(nl)) return "size mismatch";
    // header + payload == bytes, without letting a huge payload field wrap the sum
    if (h.header_bytes > bytes || h.payload != (uint64_t)(bytes - h.header_bytes))
        return "size mismatch";
    for (int i = 0; i < 9; ++i)
        if (h.dims[i] != e.dims[i]) return "size mismatch: checkpoint dimensions differ from model";
    for (int l = 0; l < nl; ++l)   // 80 + nl <= header_bytes <= bytes
        if (p[80 + l] != e.layer_types[l]) return "size mismatch: layer types differ from model";
    if (h.payload != e.nfloats * (h.dtype ? 2u : 4u)) return "size mismatch";
    if (out) *out = h;
    return nullptr;
}

void write_header(const int32_t dims[9], float eps, int32_t chunk, int32_t eos, int32_t mimo,
                  const unsigned char* layer_types, uint64_t nfloats, int f16,
                  unsigned char* p) {
    const int nl = dims[2];
    const size_t hb = header_bytes(nl);
    std::memset(p, 0, hb);
    std::memcpy(p, "SSMW", 4);
    const uint32_t ver = kVersion, dt = f16 ? 1 : 0, hb32 = (uint32_t)hb;
    const uint64_t pay = nfloats * (f16 ? 2 : 4);
    std::memcpy(p + 4, &ver, 4);
    std::memcpy(p + 8, &dt, 4);
    std::memcpy(p + 12, &hb32, 4);
    std::memcpy(p + 16, &pay, 8);
    std::memcpy(p + 24, dims, 36);
    std::memcpy(p + 60, &eps, 4);
    const int32_t g[3] = {chunk, eos, mimo};
    std::memcpy(p + 64, g, 12);
    for (int l = 0; l < nl; ++l) p[80 + l] = layer_types[l];
}

uint16_t f2h(float f) {
    uint32_t x;
    std::memcpy(&x, &f, 4);
    const uint32_t sign = (x >> 16) & 0x8000u;
    const uint32_t mag = x & 0x7fffffffu;
    if (mag >= 0x7f800000u) return (uint16_t)(sign | (mag > 0x7f800000u ? 0x7e00u : 0x7c00u));
    if (mag >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u);   // rounds to >= 65520 -> inf
    if (mag < 0x38800000u) {                                      // subnormal or zero in half
        const float af = std::fabs(f);
        const float scaled = af * 16777216.0f;                    // * 2^24: half ulp units
        return (uint16_t)(sign | (uint32_t)std::nearbyint(scaled));
    }
    const uint32_t e = ((mag >> 23) - 112) << 10;
    const uint32_t mant = mag & 0x7fffffu;
    uint32_t h = e | (mant >> 13);
    const uint32_t rest = mant & 0x1fffu;
    if (rest > 0x1000u || (rest == 0x1000u && (h & 1u))) ++h;
    return (uint16_t)(sign | h);
}

float h2f(uint16_t h) {
    const uint32_t s = (uint32_t)(h >> 15), e = (h >> 10) & 0x1f, mnt = h & 0x3ff;
    float v;
    if (e == 0) v = std::ldexp((float)mnt, -24);
    else if (e == 31) v = mnt ? NAN : INFINITY;
    else v = std::ldexp((float)(mnt | 0x400), (int)e - 25);
    return s ? -v : v;
}

void decode_payload(const unsigned char* payload, const Header& h, float* out) {
    if (h.dtype == 0) {
        std::memcpy(out, payload, (size_t)h.payload);
        return;
    }
    const size_t n = (size_t)h.payload / 2;
    for (size_t i = 0; i < n; ++i) {
        uint16_t v;
        std::memcpy(&v, payload + 2 * i, 2);
        out[i] = h2f(v);
    }
}

}  // namespace ssmw
