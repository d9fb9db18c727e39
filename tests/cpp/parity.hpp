// Test helpers for the C++ encoder-path tests: read named f32/i32 tensors from
// a baseline GGUF (the container the reference's parity baselines use,
// tests/parity.hpp:12-41) and compare element-wise (atol + rtol*|ref|) the way
// the reference's tests report, plus a relative-L2 bar.  Self-contained: a
// minimal GGUF v3 reader, no ggml.
#pragma once
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <fstream>
#include <map>
#include <string>
#include <vector>

namespace pktest {

struct GgufTensor {
    std::vector<int64_t> ne;   // ggml order (fastest first)
    uint32_t type = 0;
    uint64_t offset = 0;
};

class Gguf {
public:
    bool open(const std::string& path) {
        f_.open(path, std::ios::binary);
        if (!f_) return false;
        uint32_t magic = rd<uint32_t>(), ver = rd<uint32_t>();
        if (magic != 0x46554747u || ver < 2) return false;
        const uint64_t nt = rd<uint64_t>(), nkv = rd<uint64_t>();
        uint64_t align = 32;
        for (uint64_t i = 0; i < nkv; ++i) {
            const std::string key = rstr();
            const uint32_t t = rd<uint32_t>();
            if (key == "general.alignment" && t == 4) {
                align = rd<uint32_t>();
                continue;
            }
            skip(t);
        }
        for (uint64_t i = 0; i < nt; ++i) {
            const std::string name = rstr();
            GgufTensor g;
            const uint32_t nd = rd<uint32_t>();
            for (uint32_t d = 0; d < nd; ++d) g.ne.push_back((int64_t)rd<uint64_t>());
            g.type = rd<uint32_t>();
            g.offset = rd<uint64_t>();
            t_[name] = g;
        }
        const uint64_t pos = (uint64_t)f_.tellg();
        base_ = (pos + align - 1) / align * align;
        return (bool)f_;
    }

    // shape outermost first (slowest to fastest), like the reference's helper
    template <typename T>
    bool read(const std::string& name, uint32_t want_type, std::vector<T>& out, std::vector<int64_t>& shape) {
        auto it = t_.find(name);
        if (it == t_.end() || it->second.type != want_type) return false;
        shape.assign(it->second.ne.rbegin(), it->second.ne.rend());
        size_t n = 1;
        for (int64_t d : shape) n *= (size_t)d;
        out.resize(n);
        f_.clear();
        f_.seekg((std::streamoff)(base_ + it->second.offset));
        f_.read((char*)out.data(), (std::streamsize)(n * sizeof(T)));
        return (bool)f_;
    }

private:
    template <typename T>
    T rd() {
        T v{};
        f_.read((char*)&v, sizeof(T));
        return v;
    }
    std::string rstr() {
        const uint64_t n = rd<uint64_t>();
        std::string s(n, '\0');
        f_.read(&s[0], (std::streamsize)n);
        return s;
    }
    void skip(uint32_t t) {
        static const int sz[] = {1, 1, 2, 2, 4, 4, 4, 1, 0, 0, 8, 8, 8};
        if (t == 8) {
            rstr();
        } else if (t == 9) {
            const uint32_t et = rd<uint32_t>();
            const uint64_t n = rd<uint64_t>();
            for (uint64_t i = 0; i < n; ++i) skip(et);
        } else if (t < 13) {
            f_.seekg(sz[t], std::ios::cur);
        }
    }
    std::ifstream f_;
    std::map<std::string, GgufTensor> t_;
    uint64_t base_ = 0;
};

inline bool load_baseline(const std::string& path, const std::string& name, std::vector<float>& out,
                          std::vector<int64_t>& shape) {
    Gguf g;
    if (!g.open(path) || !g.read(name, 0u, out, shape)) {
        std::fprintf(stderr, "[parity] f32 tensor '%s' not found in %s\n", name.c_str(), path.c_str());
        return false;
    }
    return true;
}

inline bool load_baseline_i32(const std::string& path, const std::string& name, std::vector<int32_t>& out) {
    Gguf g;
    std::vector<int64_t> shape;
    if (!g.open(path) || !g.read(name, 26u, out, shape)) {
        std::fprintf(stderr, "[parity] i32 tensor '%s' not found in %s\n", name.c_str(), path.c_str());
        return false;
    }
    return true;
}

// Element-wise: |got - ref| <= atol + rtol * |ref| everywhere; prints the
// max/mean deviation and the worst element.
inline bool compare(const std::vector<float>& got, const std::vector<float>& ref, const char* label, float atol,
                    float rtol) {
    if (got.size() != ref.size()) {
        std::fprintf(stderr, "[%s] size mismatch got=%zu ref=%zu\n", label, got.size(), ref.size());
        return false;
    }
    double mx = 0, sum = 0;
    size_t worst = 0;
    bool ok = true;
    for (size_t i = 0; i < got.size(); ++i) {
        const double d = std::fabs((double)got[i] - (double)ref[i]);
        sum += d;
        if (d > mx) {
            mx = d;
            worst = i;
        }
        if (!(d <= (double)atol + (double)rtol * std::fabs((double)ref[i]))) ok = false;
    }
    std::fprintf(stderr, "[%s] n=%zu max|d|=%.3e mean|d|=%.3e (worst@%zu got=%.5f ref=%.5f) -> %s\n", label,
                 got.size(), mx, got.empty() ? 0.0 : sum / got.size(), worst, got.empty() ? 0.f : got[worst],
                 ref.empty() ? 0.f : ref[worst], ok ? "OK" : "FAIL");
    return ok;
}

// ||got - ref|| / ||ref|| <= tol.
inline bool compare_rel_l2(const std::vector<float>& got, const std::vector<float>& ref, const char* label,
                           double tol) {
    if (got.size() != ref.size()) {
        std::fprintf(stderr, "[%s] size mismatch got=%zu ref=%zu\n", label, got.size(), ref.size());
        return false;
    }
    double num = 0, den = 0;
    for (size_t i = 0; i < got.size(); ++i) {
        const double d = (double)got[i] - (double)ref[i];
        num += d * d;
        den += (double)ref[i] * ref[i];
    }
    const double r = std::sqrt(num / (den > 0 ? den : 1));
    const bool ok = r <= tol;
    std::fprintf(stderr, "[%s] rel_l2=%.3e (tol %.1e) -> %s\n", label, r, tol, ok ? "OK" : "FAIL");
    return ok;
}

// Relative-L2 bar by precision: 1e-4 for the f32 path, 1e-2 for f16/q8_0/q4_K.
inline double bar_for(int precision) { return precision == 0 ? 1e-4 : 1e-2; }

}  // namespace pktest
