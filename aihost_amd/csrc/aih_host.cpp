// aih_host.cpp -- host-side utilities of libaihost_hip.so: a deterministic
// normal generator and GGUF block quantizers, used to build synthetic GGUF
// tensors.  The reference has no quantizer (it only reads GGUF files), so these
// follow the GGUF/ggml block definitions directly; they do not need to match
// any particular quantizer bit for bit, only to produce valid blocks.
#include "../../include/aihost_hip.h"

#include <algorithm>
#include <cmath>
#include <cstring>
#include <thread>
#include <vector>

namespace {

inline uint64_t splitmix64_at(uint64_t seed, uint64_t i)
{
    uint64_t z = seed + (i + 1) * 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

// Uniform in (0, 1): 53 random bits, offset by half a step so log() is finite.
inline double uniform_at(uint64_t seed, uint64_t i)
{
    return ((double)(splitmix64_at(seed, i) >> 11) + 0.5) * (1.0 / 9007199254740992.0);
}

inline uint32_t f32_bits(float f) { uint32_t u; std::memcpy(&u, &f, 4); return u; }

// float -> IEEE binary16, round to nearest even (overflow -> inf, NaN -> qNaN).
inline uint16_t f32_to_f16(float f)
{
    uint32_t x = f32_bits(f);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t a = x & 0x7FFFFFFFu;
    if (a >= 0x7F800000u) return (uint16_t)(sign | (a > 0x7F800000u ? 0x7E00u : 0x7C00u));
    if (a >= 0x477FF000u) return (uint16_t)(sign | 0x7C00u);  // >= 65520 rounds to inf
    if (a < 0x38800000u) {                                      // below 2^-14: subnormal
        if (a < 0x33000000u) return (uint16_t)sign;             // <= 2^-25 rounds to 0
        uint32_t e = a >> 23, m = (a & 0x7FFFFFu) | 0x800000u;
        uint32_t shift = 126u - e;                              // 14..24
        uint32_t q = m >> shift, rem = m & ((1u << shift) - 1u), half = 1u << (shift - 1u);
        if (rem > half || (rem == half && (q & 1u))) ++q;
        return (uint16_t)(sign | q);
    }
    uint32_t q = (((a >> 23) - 112u) << 10) | ((a & 0x7FFFFFu) >> 13);
    uint32_t rem = a & 0x1FFFu;
    if (rem > 0x1000u || (rem == 0x1000u && (q & 1u))) ++q;
    return (uint16_t)(sign | q);
}

inline float f16_to_f32(uint16_t h)
{
    uint32_t s = (uint32_t)(h >> 15) << 31, e = (h >> 10) & 31u, m = h & 1023u;
    uint32_t bits;
    if (e == 0) {
        if (m == 0) bits = s;
        else {  // renormalise the subnormal
            int sh = 0;
            while (!(m & 0x400u)) { m <<= 1; ++sh; }
            bits = s | ((uint32_t)(113 - sh) << 23) | ((m & 0x3FFu) << 13);
        }
    } else if (e == 31) bits = s | 0x7F800000u | (m << 13);
    else bits = s | ((e + 112u) << 23) | (m << 13);
    float f; std::memcpy(&f, &bits, 4); return f;
}

inline void put_f16(uint8_t *p, float v) { uint16_t h = f32_to_f16(v); p[0] = h & 0xFF; p[1] = h >> 8; }
inline float get_f16(const uint8_t *p) { return f16_to_f32((uint16_t)(p[0] | (p[1] << 8))); }
inline int nearest_int(float v) { return (int)std::nearbyint(v); }

// GGUF Q8_0: d = absmax / 127, q = round(x / d).
void quant_q8_0(const float *x, uint8_t *b)
{
    float amax = 0.f;
    for (int j = 0; j < 32; ++j) amax = std::max(amax, std::fabs(x[j]));
    float d = amax / 127.f, id = d != 0.f ? 1.f / d : 0.f;
    put_f16(b, d);
    for (int j = 0; j < 32; ++j) b[2 + j] = (uint8_t)(int8_t)nearest_int(x[j] * id);
}

// GGUF Q4_0: d = (value of largest magnitude) / -8, q = min(15, (int8)(x/d + 8.5)).
void quant_q4_0(const float *x, uint8_t *b)
{
    float amax = 0.f, mx = 0.f;
    for (int j = 0; j < 32; ++j)
        if (std::fabs(x[j]) > amax) { amax = std::fabs(x[j]); mx = x[j]; }
    float d = mx / -8.f, id = d != 0.f ? 1.f / d : 0.f;
    put_f16(b, d);
    for (int j = 0; j < 16; ++j) {
        int q0 = std::min(15, (int)(int8_t)(x[j] * id + 8.5f));
        int q1 = std::min(15, (int)(int8_t)(x[j + 16] * id + 8.5f));
        b[2 + j] = (uint8_t)(q0 | (q1 << 4));
    }
}

// GGUF Q4_K: 8 sub-blocks of 32 with 6-bit (scale, min) pairs relative to the
// fp16 super-scales d and dmin; element = d*sc*q - dmin*mn, q in 0..15.
void quant_q4_k(const float *x, uint8_t *b)
{
    float scale[8], mins[8];
    float max_scale = 0.f, max_min = 0.f;
    for (int j = 0; j < 8; ++j) {
        float lo = 0.f, hi = x[32 * j];
        for (int i = 0; i < 32; ++i) { lo = std::min(lo, x[32 * j + i]); hi = std::max(hi, x[32 * j + i]); }
        scale[j] = (hi - lo) / 15.f;
        mins[j] = -lo;
        max_scale = std::max(max_scale, scale[j]);
        max_min = std::max(max_min, mins[j]);
    }
    float inv_scale = max_scale > 0.f ? 63.f / max_scale : 0.f;
    float inv_min = max_min > 0.f ? 63.f / max_min : 0.f;
    uint8_t *sc = b + 4;
    std::memset(sc, 0, 12);
    uint8_t ls[8], lm[8];
    for (int j = 0; j < 8; ++j) {
        ls[j] = (uint8_t)std::min(63, nearest_int(inv_scale * scale[j]));
        lm[j] = (uint8_t)std::min(63, nearest_int(inv_min * mins[j]));
        if (j < 4) {
            sc[j] = ls[j];
            sc[j + 4] = lm[j];
        } else {
            sc[j + 4] = (uint8_t)((ls[j] & 0xF) | ((lm[j] & 0xF) << 4));
            sc[j - 4] |= (uint8_t)((ls[j] >> 4) << 6);
            sc[j] |= (uint8_t)((lm[j] >> 4) << 6);
        }
    }
    put_f16(b, max_scale / 63.f);
    put_f16(b + 2, max_min / 63.f);
    float d = get_f16(b), dmin = get_f16(b + 2);
    uint8_t L[256];
    for (int j = 0; j < 8; ++j) {
        float dl = d * ls[j], dm = dmin * lm[j];
        for (int i = 0; i < 32; ++i) {
            int l = dl != 0.f ? nearest_int((x[32 * j + i] + dm) / dl) : 0;
            L[32 * j + i] = (uint8_t)std::max(0, std::min(15, l));
        }
    }
    uint8_t *qs = b + 16;
    for (int j = 0; j < 256; j += 64)
        for (int l = 0; l < 32; ++l) qs[j / 2 + l] = (uint8_t)(L[j + l] | (L[j + l + 32] << 4));
}

// GGUF Q6_K: 16 sub-blocks of 16 with int8 scales relative to the fp16 d;
// element = d*sc*(q - 32), q in 0..63 split into 4 low bits (ql) and 2 high bits (qh).
void quant_q6_k(const float *x, uint8_t *b)
{
    float scale[16];
    float max_scale = 0.f, amax_scale = 0.f;
    for (int j = 0; j < 16; ++j) {
        float amax = 0.f, mx = 0.f;
        for (int i = 0; i < 16; ++i)
            if (std::fabs(x[16 * j + i]) > amax) { amax = std::fabs(x[16 * j + i]); mx = x[16 * j + i]; }
        scale[j] = mx / -32.f;
        if (std::fabs(scale[j]) > amax_scale) { amax_scale = std::fabs(scale[j]); max_scale = scale[j]; }
    }
    uint8_t *ql = b, *qh = b + 128;
    int8_t *scales = (int8_t *)(b + 192);
    if (amax_scale == 0.f) {  // all-zero block: d = 0, every element decodes to 0
        std::memset(b, 0, 210);
        return;
    }
    float iscale = -128.f / max_scale;
    put_f16(b + 208, 1.f / iscale);
    for (int j = 0; j < 16; ++j) scales[j] = (int8_t)std::min(127, nearest_int(iscale * scale[j]));
    float d = get_f16(b + 208);
    uint8_t L[256];
    for (int j = 0; j < 16; ++j) {
        float dl = d * scales[j];
        for (int i = 0; i < 16; ++i) {
            int l = dl != 0.f ? nearest_int(x[16 * j + i] / dl) : 0;
            L[16 * j + i] = (uint8_t)(std::max(-32, std::min(31, l)) + 32);
        }
    }
    for (int j = 0; j < 256; j += 128) {
        for (int l = 0; l < 32; ++l) {
            ql[j / 2 + l] = (uint8_t)((L[j + l] & 0xF) | ((L[j + l + 64] & 0xF) << 4));
            ql[j / 2 + l + 32] = (uint8_t)((L[j + l + 32] & 0xF) | ((L[j + l + 96] & 0xF) << 4));
            qh[j / 4 + l] = (uint8_t)((L[j + l] >> 4) | ((L[j + l + 32] >> 4) << 2) |
                                      ((L[j + l + 64] >> 4) << 4) | ((L[j + l + 96] >> 4) << 6));
        }
    }
}

template <class F>
void parallel_for(int64_t n, F fn)
{
    unsigned hw = std::thread::hardware_concurrency();
    int64_t nt = std::max<int64_t>(1, std::min<int64_t>(hw ? hw : 1, 16));
    nt = std::min(nt, std::max<int64_t>(1, n / 4096));
    if (nt <= 1) { fn(0, n); return; }
    std::vector<std::thread> th;
    int64_t chunk = (n + nt - 1) / nt;
    for (int64_t t = 0; t < nt; ++t) {
        int64_t a = t * chunk, e = std::min(n, a + chunk);
        if (a < e) th.emplace_back([=] { fn(a, e); });
    }
    for (auto &t : th) t.join();
}

}  // namespace

extern "C" {

int aih_host_fill_normal(uint64_t seed, float mean, float std_, float *out, uint64_t n)
{
    if (!out && n) return AIH_E_INVALID;
    const double two_pi = 6.283185307179586476925286766559;
    uint64_t pairs = (n + 1) / 2;
    parallel_for((int64_t)pairs, [&](int64_t a, int64_t e) {
        for (int64_t p = a; p < e; ++p) {
            double u1 = uniform_at(seed, 2 * (uint64_t)p), u2 = uniform_at(seed, 2 * (uint64_t)p + 1);
            double r = std::sqrt(-2.0 * std::log(u1)), th = two_pi * u2;
            uint64_t i = 2 * (uint64_t)p;
            out[i] = (float)((double)mean + (double)std_ * r * std::cos(th));
            if (i + 1 < n) out[i + 1] = (float)((double)mean + (double)std_ * r * std::sin(th));
        }
    });
    return AIH_OK;
}

int aih_host_quantize(int type, const float *src, void *dst, int64_t n_rows, int64_t k)
{
    int qk, bytes;
    void (*fn)(const float *, uint8_t *);
    switch (type) {
    case AIH_TYPE_Q8_0: qk = 32; bytes = 34; fn = quant_q8_0; break;
    case AIH_TYPE_Q4_0: qk = 32; bytes = 18; fn = quant_q4_0; break;
    case AIH_TYPE_Q4_K: qk = 256; bytes = 144; fn = quant_q4_k; break;
    case AIH_TYPE_Q6_K: qk = 256; bytes = 210; fn = quant_q6_k; break;
    default: return AIH_E_UNSUPPORTED;
    }
    if (n_rows < 0 || k <= 0 || k % qk) return AIH_E_INVALID;
    if (!n_rows) return AIH_OK;
    if (!src || !dst) return AIH_E_INVALID;
    int64_t nb = n_rows * (k / qk);
    uint8_t *d = static_cast<uint8_t *>(dst);
    parallel_for(nb, [&](int64_t a, int64_t e) {
        for (int64_t i = a; i < e; ++i) fn(src + i * qk, d + i * bytes);
    });
    return AIH_OK;
}

}  // extern "C"
