// pkx-quantize <in.gguf> <out.gguf> <q8_0|q4_k>: the `parakeet-cli quantize`
// command (examples/cli/main.cpp:322-426) over pkx_quantize_gguf.  The
// reference also offers q4_0 / q5_0 / q5_k / q6_k; this encoder runs q8_0 and
// q4_K weights, so only those are produced.
#include <cctype>
#include <cstdio>
#include <string>

#include "pkx.h"

int main(int argc, char** argv) {
    if (argc < 4) {
        std::fprintf(stderr, "usage: pkx-quantize <in.gguf> <out.gguf> <q8_0|q4_k>\n");
        return 2;
    }
    std::string t = argv[3];
    for (char& c : t) c = (char)std::tolower((unsigned char)c);
    int gtype = -1;
    if (t == "q8_0") gtype = 8;
    else if (t == "q4_k") gtype = 12;
    if (gtype < 0) {
        std::fprintf(stderr, "pkx-quantize: unsupported type '%s' (want q8_0|q4_k)\n", argv[3]);
        return 2;
    }
    int nq = 0, nk = 0, ns = 0;
    if (pkx_quantize_gguf(argv[1], argv[2], gtype, &nq, &nk, &ns) != 0) {
        std::fprintf(stderr, "pkx-quantize: %s\n", pkx_last_error());
        return 1;
    }
    std::printf("quantize: %s -> %s [%s]\n", argv[1], argv[2], argv[3]);
    std::printf("  quantized %d tensor(s), copied %d verbatim, %d allowlisted kept F32 (block).\n", nq, nk, ns);
    return 0;
}
