// Rel-pos MHSA core: scores, rel_shift, masked softmax, attn.v, head merge.
#pragma once
#include "common.hpp"

namespace pkx {

struct AttnParams {
    const void* q = nullptr;  int64_t ldq = 0;   // [B*T][.] head h at columns h*dk
    const void* k = nullptr;  int64_t ldk = 0;
    const void* v = nullptr;  int64_t ldv = 0;
    const void* p = nullptr;  int64_t ldp = 0;   // projected pos_emb [2T-1][.]
    const float* bias_u = nullptr;               // pos_bias_u [H][dk]
    const float* bias_v = nullptr;               // pos_bias_v [H][dk]
    const int* valid = nullptr;                  // [B] valid frames per item
    void* out = nullptr;      int64_t ldo = 0;   // ctx [B*T][.]
    int B = 0, T = 0, H = 0, dk = 0;
    float scale = 1.0f;
    // chunked-limited window (relpos_attention.cpp:252-275), 0 = off: query i
    // sees key j only if 0 <= i / chunk - j / chunk <= left_chunks
    int chunk = 0, left_chunks = 0;
};

void launch_relpos_attention(Precision prec, const AttnParams& a, hipStream_t s);

}  // namespace pkx
