// Host-side helpers shared by the contexts: tensor binding against a BFW
// container, bf16 conversion, and a device arena so each context owns one
// weight allocation and one activation allocation.
#pragma once

#include "bf_model.h"
#include "hip_common.h"

#include <cmath>
#include <cstring>
#include <vector>

namespace bfhip {

// Round-to-nearest-even float -> bf16 bits, NaN kept quiet (same result as
// the device conversion).
inline uint16_t bf16_bits(float f) {
    uint32_t u;
    std::memcpy(&u, &f, 4);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

// Round-to-nearest-even float -> IEEE binary16 bits: overflow to +-Inf,
// subnormal results rounded at their own precision, NaN kept quiet.
inline uint16_t f16_bits(float f) {
    uint32_t u;
    std::memcpy(&u, &f, 4);
    const uint32_t sign = (u >> 16) & 0x8000u, a = u & 0x7fffffffu;
    if (a > 0x7f800000u) return (uint16_t)(sign | 0x7e00u);
    if (a >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u);  // rounds past 65504
    if (a >= 0x38800000u) {                                    // normal binary16
        const uint32_t r = a + 0x0fffu + ((a >> 13) & 1u);
        return (uint16_t)(sign | ((r - 0x38000000u) >> 13));
    }
    if (a < 0x33000000u) return (uint16_t)sign;                // below half the least subnormal
    const uint32_t e = a >> 23, m = (a & 0x7fffffu) | 0x800000u;
    const uint32_t shift = 126u - e;                          // 14..24 for this range
    const uint32_t half = 1u << (shift - 1), rest = m & ((1u << shift) - 1u);
    uint32_t q = m >> shift;
    if (rest > half || (rest == half && (q & 1u))) ++q;
    return (uint16_t)(sign | q);
}

// IEEE binary16 bits -> float (exact).
inline float f16_value(uint16_t h) {
    const uint32_t e = (h >> 10) & 0x1fu, m = h & 0x3ffu;
    float v;
    if (e == 0) v = std::ldexp((float)m, -24);
    else if (e == 31) v = m ? NAN : INFINITY;
    else v = std::ldexp((float)(m | 0x400u), (int)e - 25);
    return (h & 0x8000u) ? -v : v;
}

// Looks a tensor up by name and checks dtype, rank and every dimension
// (the binding contract of reference cuda_swin.cu:57-63).
inline const void *bind_tensor(const bf_model *m, const char *name, uint32_t dtype,
                               uint32_t rank, const uint32_t *dims, char *error, size_t cap) {
    const bf_tensor *t = bf_model_find(m, name);
    if (!t) return fail(error, cap, "missing tensor %s", name), nullptr;
    if (t->dtype != dtype || t->rank != rank)
        return fail(error, cap, "%s: dtype/rank mismatch", name), nullptr;
    for (uint32_t i = 0; i < rank; ++i)
        if (t->dims[i] != dims[i])
            return fail(error, cap, "%s: dimension %u is %u, expected %u", name, i, t->dims[i],
                        dims[i]),
                   nullptr;
    return t->data;
}

inline const float *bind_f32(const bf_model *m, const char *name,
                             std::initializer_list<uint32_t> dims, char *error, size_t cap) {
    std::vector<uint32_t> d(dims);
    return (const float *)bind_tensor(m, name, BF_DTYPE_F32, (uint32_t)d.size(), d.data(), error,
                                      cap);
}

// Staging area for one context's parameters: host bytes are appended with
// 256-byte alignment, then uploaded in a single copy; offsets become device
// pointers afterwards.
struct ParamArena {
    std::vector<unsigned char> host;
    size_t add(const void *src, size_t bytes) {
        const size_t off = (host.size() + 255) & ~size_t(255);
        host.resize(off + bytes);
        if (src) std::memcpy(host.data() + off, src, bytes);
        return off;
    }
    size_t add_f32(const float *src, size_t count) { return add(src, count * 4); }
    size_t add_bf16(const float *src, size_t count) {
        std::vector<uint16_t> tmp(count);
        for (size_t i = 0; i < count; ++i) tmp[i] = bf16_bits(src[i]);
        return add(tmp.data(), count * 2);
    }
    size_t add_f16(const float *src, size_t count) {
        std::vector<uint16_t> tmp(count);
        for (size_t i = 0; i < count; ++i) tmp[i] = f16_bits(src[i]);
        return add(tmp.data(), count * 2);
    }
    size_t add_f32(const std::vector<float> &v) { return add_f32(v.data(), v.size()); }
    size_t add_bf16(const std::vector<float> &v) { return add_bf16(v.data(), v.size()); }
    size_t add_f16(const std::vector<float> &v) { return add_f16(v.data(), v.size()); }
};

}  // namespace bfhip
