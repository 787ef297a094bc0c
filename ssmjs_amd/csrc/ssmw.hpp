// SSMW checkpoint images (the weight format of ssm_model_export_weights / load_weights): header
// layout, validation against a model's dimensions and the f16 payload codec. Host-only C++ (no
// HIP): built into the library with the host compiler, and on its own under AddressSanitizer
// and UndefinedBehaviorSanitizer by the CPU tests, which feed it truncated, oversized and
// corrupted images.
//
// Header (little endian, header_bytes(n_layers) long, 16-byte aligned):
//   0   "SSMW"              4   version (1)          8   dtype (0 f32, 1 f16)
//   12  header bytes        16  payload bytes (u64)
//   24  vocab, d_model, n_layers, d_state, d_conv, expand, n_heads, n_groups, dt_rank (i32)
//   60  norm eps (f32)      64  chunk_len, eos_id, mimo_group (i32), 76 reserved
//   80  one layer-type byte per layer, zero padding to header_bytes
// then the payload: the model's weights in payload order, f32 or f16.
#pragma once

#include <cstddef>
#include <cstdint>

namespace ssmw {

constexpr uint32_t kVersion = 1;

inline size_t header_bytes(int n_layers) {
    return 80 + (size_t)((n_layers + 15) / 16) * 16;
}

struct Header {
    uint32_t version, dtype, header_bytes;
    uint64_t payload;
    int32_t dims[9];   // vocab, d_model, n_layers, d_state, d_conv, expand, n_heads, n_groups, dt_rank
    float eps;
    int32_t chunk, eos, mimo;
};

// What an image must match to load into a model.
struct Expect {
    int32_t dims[9];
    const unsigned char* layer_types;   // n_layers = dims[2] bytes
    uint64_t nfloats;                   // payload elements
};

// Validate `bytes` bytes at `buf` against `e`: nullptr if the image loads, otherwise the
// reason ("bad magic", "unsupported version", "unsupported dtype", "size mismatch...").
// Reads nothing outside [buf, buf + bytes).
const char* validate(const void* buf, size_t bytes, const Expect& e, Header* out);

// Header of an image for a model with dims / layer types and `nfloats` weights.
void write_header(const int32_t dims[9], float eps, int32_t chunk, int32_t eos, int32_t mimo,
                  const unsigned char* layer_types, uint64_t nfloats, int f16,
                  unsigned char* out);

// IEEE binary16 <-> binary32, round to nearest even.
uint16_t f2h(float f);
float h2f(uint16_t h);

// The validated payload as floats (f32 copied, f16 widened): out holds h.payload / element size.
void decode_payload(const unsigned char* payload, const Header& h, float* out);

}  // namespace ssmw
