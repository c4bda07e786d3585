// quantize.cpp - host-side fp32 -> block quantizers for synthetic expert
// weights (Q8_0, Q4_K, Q5_K, Q6_K).
//
// The reference has no quantizer: it only reads GGUF files produced elsewhere.
// These encoders are our own simple min/max schemes; any valid encoding is
// acceptable because parity is always checked on the very same bytes.  The
// byte layouts are the ones the reference decodes (qwen3moe.cpp:128-202).
#include <stdint.h>
#include <string.h>

#include <algorithm>
#include <cmath>
#include <thread>
#include <vector>

#include "../../include/eahmmf_hip.h"

namespace {

// float -> IEEE half, round to nearest even.
uint16_t to_half(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    const uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t mant = x & 0x7FFFFFu;
    const int exp = (int)((x >> 23) & 0xFFu);
    if (exp == 0xFF) return (uint16_t)(sign | 0x7C00u | (mant ? 0x200u : 0u));
    const int e = exp - 127 + 15;
    if (e >= 31) return (uint16_t)(sign | 0x7C00u);
    if (e <= 0) {
        if (e < -10) return (uint16_t)sign;
        mant |= 0x800000u;
        const int shift = 14 - e;
        uint32_t hm = mant >> shift;
        const uint32_t rem = mant & ((1u << shift) - 1u), half = 1u << (shift - 1);
        if (rem > half || (rem == half && (hm & 1u))) hm++;
        return (uint16_t)(sign | hm);
    }
    uint32_t out = sign | ((uint32_t)e << 10) | (mant >> 13);
    const uint32_t rem = mant & 0x1FFFu;
    if (rem > 0x1000u || (rem == 0x1000u && (out & 1u))) out++;
    return (uint16_t)out;
}

float from_half(uint16_t h) {
    const uint32_t s = (h >> 15) & 1u, e = (h >> 10) & 31u, m = h & 1023u;
    float v;
    if (e == 0) v = ldexpf((float)m, -24);
    else if (e == 31) v = m ? NAN : INFINITY;
    else v = ldexpf((float)(m | 1024u), (int)e - 25);
    return s ? -v : v;
}

int clampi(int v, int lo, int hi) { return v < lo ? lo : (v > hi ? hi : v); }

void q8_0_block(const float* x, uint8_t* b) {
    float amax = 0.f;
    for (int i = 0; i < 32; i++) amax = std::max(amax, std::fabs(x[i]));
    const uint16_t dh = to_half(amax / 127.f);
    b[0] = (uint8_t)(dh & 0xFF);
    b[1] = (uint8_t)(dh >> 8);
    const float d = from_half(dh), id = d > 0.f ? 1.f / d : 0.f;
    for (int i = 0; i < 32; i++) b[2 + i] = (uint8_t)(int8_t)clampi((int)lrintf(x[i] * id), -127, 127);
}

// Packs eight 6-bit (scale, min) pairs the way scale_min_k4 unpacks them
// (qwen3moe.cpp:133-141).
void pack_scale_min(const int* sc, const int* mn, uint8_t* q) {
    for (int j = 0; j < 4; j++) {
        q[j] = (uint8_t)((sc[j] & 63) | ((sc[j + 4] >> 4) << 6));
        q[j + 4] = (uint8_t)((mn[j] & 63) | ((mn[j + 4] >> 4) << 6));
        q[j + 8] = (uint8_t)((sc[j + 4] & 15) | ((mn[j + 4] & 15) << 4));
    }
}

// Q4_K (nlev = 15) and Q5_K (nlev = 31): y = d*sc*q - dmin*m per 32-value sub-block.
void qk_block(const float* x, uint8_t* b, int nlev) {
    float scale[8], minv[8];
    float maxs = 0.f, maxm = 0.f;
    for (int j = 0; j < 8; j++) {
        float lo = x[32 * j], hi = x[32 * j];
        for (int i = 1; i < 32; i++) {
            lo = std::min(lo, x[32 * j + i]);
            hi = std::max(hi, x[32 * j + i]);
        }
        lo = std::min(lo, 0.f);
        scale[j] = (hi - lo) / (float)nlev;
        minv[j] = -lo;
        maxs = std::max(maxs, scale[j]);
        maxm = std::max(maxm, minv[j]);
    }
    const uint16_t dh = to_half(maxs / 63.f), mh = to_half(maxm / 63.f);
    const float d = from_half(dh), dmin = from_half(mh);
    int sc[8], mn[8];
    for (int j = 0; j < 8; j++) {
        sc[j] = d > 0.f ? clampi((int)lrintf(scale[j] / d), 0, 63) : 0;
        mn[j] = dmin > 0.f ? clampi((int)lrintf(minv[j] / dmin), 0, 63) : 0;
    }
    b[0] = (uint8_t)(dh & 0xFF); b[1] = (uint8_t)(dh >> 8);
    b[2] = (uint8_t)(mh & 0xFF); b[3] = (uint8_t)(mh >> 8);
    pack_scale_min(sc, mn, b + 4);
    int q[256];
    for (int j = 0; j < 8; j++) {
        const float ds = d * (float)sc[j], dm = dmin * (float)mn[j];
        for (int i = 0; i < 32; i++)
            q[32 * j + i] = ds > 0.f ? clampi((int)lrintf((x[32 * j + i] + dm) / ds), 0, nlev) : 0;
    }
    uint8_t* qs = b + (nlev == 15 ? 16 : 48);
    if (nlev == 31) memset(b + 16, 0, 32);
    for (int g = 0; g < 4; g++)
        for (int l = 0; l < 32; l++) {
            const int a = q[64 * g + l], c = q[64 * g + 32 + l];
            qs[32 * g + l] = (uint8_t)((a & 15) | ((c & 15) << 4));
            if (nlev == 31) {
                b[16 + l] |= (uint8_t)(((a >> 4) & 1) << (2 * g));
                b[16 + l] |= (uint8_t)(((c >> 4) & 1) << (2 * g + 1));
            }
        }
}

// Q6_K: sixteen 16-value groups with int8 scales and one fp16 d.
void q6_k_block(const float* x, uint8_t* b) {
    float scale[16], maxs = 0.f;
    for (int g = 0; g < 16; g++) {
        float amax = 0.f;
        for (int i = 0; i < 16; i++) amax = std::max(amax, std::fabs(x[16 * g + i]));
        scale[g] = amax / 31.f;
        maxs = std::max(maxs, scale[g]);
    }
    const uint16_t dh = to_half(maxs / 127.f);
    const float d = from_half(dh);
    memset(b, 0, 210);
    int8_t* sc = (int8_t*)(b + 192);
    int q[256];
    for (int g = 0; g < 16; g++) {
        sc[g] = (int8_t)(d > 0.f ? clampi((int)lrintf(scale[g] / d), -128, 127) : 0);
        const float ds = d * (float)sc[g];
        for (int i = 0; i < 16; i++)
            q[16 * g + i] = ds > 0.f ? clampi((int)lrintf(x[16 * g + i] / ds), -32, 31) : 0;
    }
    for (int n = 0; n < 2; n++)
        for (int u = 0; u < 4; u++)
            for (int l = 0; l < 32; l++) {
                const int v = q[128 * n + 32 * u + l] + 32;
                uint8_t& lo = b[64 * n + l + 32 * (u & 1)];
                lo |= (uint8_t)((v & 15) << (u < 2 ? 0 : 4));
                b[128 + 32 * n + l] |= (uint8_t)(((v >> 4) & 3) << (2 * u));
            }
    b[208] = (uint8_t)(dh & 0xFF);
    b[209] = (uint8_t)(dh >> 8);
}

}  // namespace

extern "C" size_t eahmmf_hip_row_bytes(int type, int64_t ne0) {
    int blck = 0, bytes = 0;
    switch (type) {
        case 0: blck = 32; bytes = 128; break;
        case 8: blck = 32; bytes = 34; break;
        case 12: blck = 256; bytes = 144; break;
        case 13: blck = 256; bytes = 176; break;
        case 14: blck = 256; bytes = 210; break;
        default: return 0;
    }
    if (ne0 <= 0 || ne0 % blck) return 0;
    return (size_t)(ne0 / blck) * (size_t)bytes;
}

extern "C" int64_t eahmmf_hip_quantize_rows(int type, const float* src, int64_t nrows, int64_t ne0, uint8_t* dst) {
    const size_t rb = eahmmf_hip_row_bytes(type, ne0);
    if (!rb || !src || !dst || nrows < 0 || type == 0) return -1;
    auto work = [&](int64_t r0, int64_t r1) {
        for (int64_t r = r0; r < r1; r++) {
            const float* x = src + (size_t)r * ne0;
            uint8_t* o = dst + (size_t)r * rb;
            switch (type) {
                case 8:
                    for (int64_t b = 0; b < ne0 / 32; b++) q8_0_block(x + 32 * b, o + 34 * b);
                    break;
                case 12:
                    for (int64_t b = 0; b < ne0 / 256; b++) qk_block(x + 256 * b, o + 144 * b, 15);
                    break;
                case 13:
                    for (int64_t b = 0; b < ne0 / 256; b++) qk_block(x + 256 * b, o + 176 * b, 31);
                    break;
                case 14:
                    for (int64_t b = 0; b < ne0 / 256; b++) q6_k_block(x + 256 * b, o + 210 * b);
                    break;
            }
        }
    };
    const unsigned hw = std::max(1u, std::min(16u, std::thread::hardware_concurrency()));
    const int64_t nthr = std::min<int64_t>(hw, std::max<int64_t>(1, nrows / 64));
    if (nthr <= 1) {
        work(0, nrows);
    } else {
        std::vector<std::thread> th;
        const int64_t per = (nrows + nthr - 1) / nthr;
        int64_t started = 0;  // rows [0, started) are handed to threads
        try {
            for (int64_t t = 0; t < nthr; t++) {
                const int64_t a = t * per, z = std::min(nrows, a + per);
                if (a < z) th.emplace_back(work, a, z);
                started = std::max(started, z);
            }
        } catch (...) {
            // a thread could not be started: the remaining rows are quantized
            // on this thread (no exception leaves the C ABI)
        }
        if (started < nrows) work(started, nrows);
        for (auto& t : th) t.join();
    }
    return (int64_t)(rb * (size_t)nrows);
}
