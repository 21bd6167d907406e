// Synthetic inputs of the benchmark configurations and the blob format.
//
// Random streams use the reference's xorshift64 (crates/llmpager-bench/src/
// main.rs:99-120: x ^= x<<13; x ^= x>>7; x ^= x<<17; unit = (x>>11)/2^53),
// one independent stream per (seed, tag...) whose start state is a splitmix64
// hash of the tag, so every blob / tensor can be generated on its own thread
// and the result does not depend on threading.  Normals are Box-Muller
// (first output of each pair).
#include <math.h>
#include <string.h>

#include <cstdint>

#include "../../include/llmpager_hip.h"

namespace {

uint64_t splitmix64(uint64_t x) {
    x += 0x9e3779b97f4a7c15ull;
    x = (x ^ (x >> 30)) * 0xbf58476d1ce4e5b9ull;
    x = (x ^ (x >> 27)) * 0x94d049bb133111ebull;
    return x ^ (x >> 31);
}

struct Xorshift {
    uint64_t s;
    explicit Xorshift(uint64_t seed, uint64_t a, uint64_t b = 0, uint64_t c = 0) {
        uint64_t h = splitmix64(seed);
        h = splitmix64(h ^ a);
        h = splitmix64(h ^ b);
        h = splitmix64(h ^ c);
        s = h ? h : 1;  // xorshift state must be nonzero (main.rs:103-105)
    }
    uint64_t next() {
        uint64_t x = s;
        x ^= x << 13;
        x ^= x >> 7;
        x ^= x << 17;
        s = x;
        return x;
    }
    double unit() { return (double)(next() >> 11) / 9007199254740992.0; }
    double normal() {
        double u1 = unit(), u2 = unit();
        if (u1 <= 0.0) u1 = 1.0 / 9007199254740992.0;
        return sqrt(-2.0 * log(u1)) * cos(6.283185307179586 * u2);
    }
};

uint32_t f2u(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    return u;
}

// IEEE round-to-nearest-even f32 -> f16 bits (finite, non-negative inputs
// below 65504 here).
uint16_t f16_rne(float x) {
    uint32_t b = f2u(x);
    uint16_t sign = (uint16_t)((b >> 16) & 0x8000u);
    uint32_t a = b & 0x7fffffffu;
    if (a >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u);
    if (a < 0x38800000u) {
        if (a < 0x33000000u) return sign;
        uint32_t e = a >> 23;
        uint32_t m = (a & 0x7fffffu) | 0x800000u;
        uint32_t shift = 126 - e;
        uint32_t q = m >> shift;
        uint32_t rem = m & ((1u << shift) - 1u);
        uint32_t half = 1u << (shift - 1);
        if (rem > half || (rem == half && (q & 1u))) q++;
        return (uint16_t)(sign | q);
    }
    uint32_t r = a + 0xfffu + ((a >> 13) & 1u);
    r -= 0x38000000u;
    return (uint16_t)(sign | (r >> 13));
}

uint16_t bf16_rne(float f) {
    uint32_t b = f2u(f);
    return (uint16_t)((b + 0x7fffu + ((b >> 16) & 1u)) >> 16);
}

void put_u32(uint8_t* p, uint32_t v) { memcpy(p, &v, 4); }

// One q4 region [rows, cols]: f16 scales |N(0, 0.02)|/8, nibbles uniform.
void synth_region(uint8_t* dst, int rows, int cols, int group, Xorshift& rng) {
    const size_t ns = (size_t)rows * (cols / group);
    for (size_t i = 0; i < ns; ++i) {
        const float s = (float)(fabs(rng.normal() * 0.02) / 8.0);
        const uint16_t h = f16_rne(s);
        memcpy(dst + 2 * i, &h, 2);
    }
    uint8_t* data = dst + 2 * ns;
    const size_t nb = (size_t)rows * cols / 2;
    size_t i = 0;
    for (; i + 8 <= nb; i += 8) {
        const uint64_t r = rng.next();
        memcpy(data + i, &r, 8);
    }
    if (i < nb) {
        const uint64_t r = rng.next();
        memcpy(data + i, &r, nb - i);
    }
}

}  // namespace

extern "C" {

uint64_t lp_q4_bytes(int rows, int cols, int group) {
    return (uint64_t)rows * (uint64_t)(cols / group) * 2 + (uint64_t)rows * (uint64_t)cols / 2;
}

uint64_t lp_blob_bytes(int hidden, int inter, int group) {
    return 32 + 2 * lp_q4_bytes(inter, hidden, group) + lp_q4_bytes(hidden, inter, group);
}

void lp_blob_offsets(int hidden, int inter, int group, uint64_t* gate_off, uint64_t* up_off,
                     uint64_t* down_off) {
    const uint64_t gb = lp_q4_bytes(inter, hidden, group);
    if (gate_off) *gate_off = 32;
    if (up_off) *up_off = 32 + gb;
    if (down_off) *down_off = 32 + 2 * gb;
}

int lp_synth_blob(uint8_t* dst, int hidden, int inter, int group, uint64_t seed, int layer,
                  int expert) {
    if (!dst || hidden <= 0 || inter <= 0 || group <= 0 || hidden % group || inter % group)
        return LP_E_INVALID;
    // Header: gate, up, down as (rows, cols) u32 pairs, then group, then 0
    // (crates/llmpager-convert/src/lib.rs:276-281).
    const uint32_t hdr[8] = {(uint32_t)inter, (uint32_t)hidden, (uint32_t)inter, (uint32_t)hidden,
                             (uint32_t)hidden, (uint32_t)inter, (uint32_t)group, 0u};
    for (int i = 0; i < 8; ++i) put_u32(dst + 4 * i, hdr[i]);
    uint64_t go, uo, dn;
    lp_blob_offsets(hidden, inter, group, &go, &uo, &dn);
    Xorshift rng(seed, 0x5e11ull, (uint64_t)layer, (uint64_t)expert);
    synth_region(dst + go, inter, hidden, group, rng);
    synth_region(dst + uo, inter, hidden, group, rng);
    synth_region(dst + dn, hidden, inter, group, rng);
    return LP_OK;
}

int lp_synth_blobs(uint8_t* dst, uint64_t stride, int n, int hidden, int inter, int group,
                   uint64_t seed, int layer, int e0, int threads) {
    if (!dst || n < 0 || stride < lp_blob_bytes(hidden, inter, group)) return LP_E_INVALID;
    int bad = 0;
#pragma omp parallel for num_threads(threads > 0 ? threads : 1) schedule(dynamic, 1) reduction(| : bad)
    for (int i = 0; i < n; ++i)
        bad |= lp_synth_blob(dst + (uint64_t)i * stride, hidden, inter, group, seed, layer, e0 + i) != LP_OK;
    return bad ? LP_E_INVALID : LP_OK;
}

int lp_synth_bf16(uint16_t* dst, uint64_t n, float std_dev, uint64_t seed, uint64_t stream) {
    if (!dst) return LP_E_INVALID;
    Xorshift rng(seed, 0xbf16ull, stream);
    for (uint64_t i = 0; i < n; ++i) dst[i] = bf16_rne((float)(rng.normal() * std_dev));
    return LP_OK;
}

int lp_synth_f32_bf16(float* dst, uint64_t n, float std_dev, uint64_t seed, uint64_t stream) {
    if (!dst) return LP_E_INVALID;
    Xorshift rng(seed, 0xf32ull, stream);
    for (uint64_t i = 0; i < n; ++i) {
        const uint32_t b = (uint32_t)bf16_rne((float)(rng.normal() * std_dev)) << 16;
        memcpy(dst + i, &b, 4);
    }
    return LP_OK;
}

}  // extern "C"
