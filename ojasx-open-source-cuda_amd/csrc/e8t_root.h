// e8t_root.h -- the 1-bit Root-E8 table (RootE8LatticePacker, lattice.py:426-533).
//
// 256 entries of 8 coordinates, as the reference builds them (lattice.py:436-456) and
// scales them by 2:
//   0..111   +-2 at i and +-2 at j (i < j), loops i, j, s1 in (-, +), s2 in (-, +)
//   112..239 (+-1)^8 with an even number of -1, in itertools.product order over (-, +)
//            with the first coordinate slowest: entry 112 + P for the 7-bit prefix P of
//            the sign bits (bit 6 - k = 1 for + at coordinate k), the last sign fixing
//            the parity
//   240..255 +-2 at i, loops i, s in (-, +)
// The table is generated at compile time.
#pragma once

#include <stdint.h>

#include "e8t_device.h"

namespace ojx {

struct RootTable {
    int8_t c[256][8];
};

constexpr RootTable make_root_table() {
    RootTable t{};
    int e = 0;
    for (int i = 0; i < 8; ++i)
        for (int j = i + 1; j < 8; ++j)
            for (int a = 0; a < 2; ++a)
                for (int b = 0; b < 2; ++b) {
                    t.c[e][i] = (int8_t)(a ? 2 : -2);
                    t.c[e][j] = (int8_t)(b ? 2 : -2);
                    ++e;
                }
    for (int p = 0; p < 256; ++p) {
        int neg = 0;
        for (int k = 0; k < 8; ++k) neg += ((p >> (7 - k)) & 1) ? 0 : 1;
        if (neg & 1) continue;
        for (int k = 0; k < 8; ++k) t.c[e][k] = (int8_t)(((p >> (7 - k)) & 1) ? 1 : -1);
        ++e;
    }
    for (int i = 0; i < 8; ++i)
        for (int s = 0; s < 2; ++s) {
            t.c[e][i] = (int8_t)(s ? 2 : -2);
            ++e;
        }
    return t;
}

constexpr RootTable kRootTableHost = make_root_table();
static_assert(kRootTableHost.c[0][0] == -2 && kRootTableHost.c[0][1] == -2, "entry 0");
static_assert(kRootTableHost.c[112][0] == -1 && kRootTableHost.c[112][7] == -1, "entry 112");
static_assert(kRootTableHost.c[239][0] == 1 && kRootTableHost.c[239][7] == 1, "entry 239");
static_assert(kRootTableHost.c[255][7] == 2, "entry 255");

// Device copy (read through the vector caches; 2 KB).
__device__ __constant__ const RootTable kRootTable = make_root_table();

// Decoded 1-bit weight under the reference's dtype rule (lattice.py:528-533):
// table[code][k] * scales.to(dtype), computed in fp32 (exact) and rounded once to dtype
// (fp16 can overflow to inf for |2 s| > 65504, as the reference's fp16 product does).
template <int DT> __device__ __forceinline__ float deq1_value(uint32_t code, int k, uint32_t s16) {
    float p = (float)kRootTable.c[code][k] * scale_for<DT>(s16);
    keep_f32(p);
    if constexpr (DT == kF16) return f16_bits_to_f32(f32_to_f16_bits(p));
    else if constexpr (DT == kBF16) return bf16_bits_to_f32(f32_to_bf16_bits(p));
    else return p;
}

// v_perm_b32 selector bytes of a coordinate against the 8-byte value table
// {S0 = +s | +2s << 16, S1 = -s | -2s << 16} (S1 holds bytes 0..3): 12 selects 0x00.
constexpr uint32_t root_sel_pair(int c) {
    return c == 0 ? 0x0C0Cu : c == 1 ? 0x0504u : c == 2 ? 0x0706u : c == -1 ? 0x0100u : 0x0302u;
}

// Code of one 8-vector v (already divided by the group's initial scale): argmax over the
// 256 rows u of v . u/|u| as RootE8LatticePacker.pack evaluates it (lattice.py:497-500).
// Each dot product is torch's CPU matmul chain acc = fma(v_k, u_k, acc) from +0 over
// k = 0..7; with the table's zeros that chain is, exactly:
//   rows +-2 at i, j:   fma(v_j, +-c1, +-rnd(c1 v_i))          c1 = 2 / sqrt(8) in fp32
//   rows (+-1)^8:       the full chain with +-c2 = +-1 / sqrt(8)
//   rows +-2 at i:      +-v_i                                  (2 / 2 = 1)
// The (+-1)^8 rows come in negated pairs (same parity): rows 112 + P and 112 + 127 - P,
// and a chain with every sign flipped is the exact negation, so the 64 chains with a
// negative first coordinate give all 128 dots (a 7-level prefix tree, 190 FMAs).  The
// candidates are compared in table order with a strict > (the first maximum wins, as
// torch.argmax).
__host__ __device__ inline uint32_t root_code(const float (&v)[8]) {
#pragma clang fp contract(off)
    const float n8 = __builtin_sqrtf(8.0f);
    const float c1 = 2.0f / n8, c2 = 1.0f / n8;
    float best = 0.f;
    uint32_t bi = 0;
    // rows 0..111: pairs (i, j), signs (s1, s2) in (-,-), (-,+), (+,-), (+,+)
    float t[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) t[i] = __builtin_fmaf(v[i], c1, 0.f);
    uint32_t e = 0;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
#pragma unroll
        for (int j = i + 1; j < 8; ++j) {
#pragma unroll
            for (int a = 0; a < 2; ++a) {
#pragma unroll
                for (int b = 0; b < 2; ++b) {
                    const float d = __builtin_fmaf(v[j], b ? c1 : -c1, a ? t[i] : -t[i]);
                    if (e == 0 || d > best) {
                        best = d;
                        bi = e;
                    }
                    ++e;
                }
            }
        }
    }
    // rows 112..239: chains of the 64 prefixes with a negative first coordinate
    float leaf[64];
    {
        float l0 = __builtin_fmaf(v[0], -c2, 0.f);
        float l1[2], l2[4], l3[8], l4[16], l5[32];
#pragma unroll
        for (int b = 0; b < 2; ++b) l1[b] = __builtin_fmaf(v[1], b ? c2 : -c2, l0);
#pragma unroll
        for (int q = 0; q < 4; ++q) l2[q] = __builtin_fmaf(v[2], (q & 1) ? c2 : -c2, l1[q >> 1]);
#pragma unroll
        for (int q = 0; q < 8; ++q) l3[q] = __builtin_fmaf(v[3], (q & 1) ? c2 : -c2, l2[q >> 1]);
#pragma unroll
        for (int q = 0; q < 16; ++q) l4[q] = __builtin_fmaf(v[4], (q & 1) ? c2 : -c2, l3[q >> 1]);
#pragma unroll
        for (int q = 0; q < 32; ++q) l5[q] = __builtin_fmaf(v[5], (q & 1) ? c2 : -c2, l4[q >> 1]);
#pragma unroll
        for (int q = 0; q < 64; ++q) {
            const float l6 = __builtin_fmaf(v[6], (q & 1) ? c2 : -c2, l5[q >> 1]);
            // negatives so far: 1 (coordinate 0) + zero bits of q (coordinates 1..6); the
            // last coordinate makes the count even
            const int neg = 1 + (6 - __builtin_popcount((unsigned)q));
            leaf[q] = __builtin_fmaf(v[7], (neg & 1) ? -c2 : c2, l6);
        }
    }
#pragma unroll
    for (int P = 0; P < 128; ++P) {
        const float d = P < 64 ? leaf[P] : -leaf[127 - P];
        if (d > best) {
            best = d;
            bi = 112u + (uint32_t)P;
        }
    }
    // rows 240..255: +-2 at i
#pragma unroll
    for (int i = 0; i < 8; ++i) {
#pragma unroll
        for (int s = 0; s < 2; ++s) {
            const float d = s ? v[i] : -v[i];
            if (d > best) {
                best = d;
                bi = 240u + 2u * (uint32_t)i + (uint32_t)s;
            }
        }
    }
    return bi;
}


// 1-bit value words and v_perm_b32 selectors: per scale group the weights +-s and +-rnd(2s)
// in the activation dtype, S0 = s | rnd(2s) << 16, S1 = -s | -rnd(2s) << 16; a 256-entry
// table (4 KB) maps a code to the four selector words of its 8 weights.
constexpr int kSel1Entries = 256;

__device__ __forceinline__ void fill_sel1(uint4* tab, int nthreads) {
    for (int e = (int)threadIdx.x; e < kSel1Entries; e += nthreads) {
        uint32_t w[4];
#pragma unroll
        for (int h = 0; h < 4; ++h)
            w[h] = root_sel_pair(kRootTable.c[e][2 * h]) |
                   (root_sel_pair(kRootTable.c[e][2 * h + 1]) << 16);
        tab[e] = make_uint4(w[0], w[1], w[2], w[3]);
    }
}

template <int DT>
__device__ __forceinline__ uint2 values1(uint32_t s16) {
    const float s = scale_for<DT>(s16 & 0xFFFFu);
    const uint32_t a = rnd_bits<DT>(s), b = rnd_bits<DT>(2.0f * s);
    return make_uint2(a | (b << 16), (a ^ 0x8000u) | ((b ^ 0x8000u) << 16));
}

}  // namespace ojx
