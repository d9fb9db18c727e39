// Weight quantisation (ggml_quantize_chunk for q8_0 / q4_K) and the GGUF
// quantiser of parakeet-cli quantize (examples/cli/main.cpp:279-426).
#pragma once
#include <hip/hip_runtime.h>

#include <cstdint>
#include <string>

namespace pkx {

// x [rows][per_row] f32 (device) -> y: rows of ggml blocks (device).
void quantize_rows(int gtype, const float* x, void* y, int64_t rows, int64_t per_row, hipStream_t s);

// The allowlist of quantisable tensor names (examples/cli/main.cpp:279-303).
bool is_quantizable_name(const std::string& n);

struct QuantizeCounts {
    int quantized = 0, kept = 0, skipped = 0;
};
// Copies every KV pair verbatim, quantises the allowlisted f32 2-D tensors
// whose row length divides into blocks (on the device), copies the rest.
QuantizeCounts quantize_gguf(const std::string& in_path, const std::string& out_path, int gtype);

}  // namespace pkx
