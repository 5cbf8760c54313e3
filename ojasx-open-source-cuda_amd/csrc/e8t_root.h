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


// The full search out of line: its 64 partial chains stay out of the callers' registers.
__host__ __device__ __attribute__((noinline)) inline uint32_t root_code_full(const float (&v)[8]) {
    return root_code(v);
}

// root_code with the same result from a handful of candidate rows.  Per row family the best
// exact-arithmetic dot (constants c1 = 2 c2 as above; a_k = |v_k|, S = sum a_k) is known in
// closed form, and so is the runner-up:
//   rows +-2 at i, j:  c1 (a_i + a_j) with signs matching v: best pair (1st, 2nd largest a),
//                      then (1st, 3rd); every other row <= c1 max(m2 + m3, m1 + m4)
//   rows (+-1)^8:      c2 (S - 2 sum_F a) over flip sets F of the parity that keeps an even
//                      number of minus signs: F = {} or {smallest}, then {two smallest} or
//                      {second smallest}; every other row <= c2 (S - 2 (a(1) + a(3))) or
//                      c2 (S - 2 a(3))
//   rows +-2 at i:     a_i: largest, then second largest; every other row <= m3
// (m1 >= m2 >= ... the largest, a(1) <= a(2) <= ... the smallest magnitudes).  The six
// candidates' dots are evaluated as the reference's fp32 chains (exactly as root_code does)
// and the largest wins, the lower row index on ties.  That is the reference's argmax when the
// winner exceeds the bound on all other rows by more than the chains' rounding error (at
// most ~2^-16 (1 + S)): the margin used is 2^-12 (1 + S).  Otherwise (near-ties of three
// rows, zero vectors) the full search runs.  Magnitudes are ordered by a 19-comparator
// sorting network on keys whose low 3 bits hold the coordinate (order ties are harmless:
// the bounds absorb them), the exact magnitudes of the chosen coordinates recovered from
// the keys and a word of the dropped low bits.
__host__ __device__ inline uint32_t root_code_fast(const float (&v)[8]) {
#pragma clang fp contract(off)
    const float n8 = __builtin_sqrtf(8.0f);
    const float c1 = 2.0f / n8, c2 = 1.0f / n8;
    float a[8];
    uint32_t key[8];
    uint32_t low = 0u, neg = 0u;  // low bits of a_k (3 per k); bit k: v_k < 0
    float S = 0.f;
#pragma unroll
    for (int k = 0; k < 8; ++k) {
        a[k] = __builtin_fabsf(v[k]);
        uint32_t bits;
        __builtin_memcpy(&bits, &a[k], 4);
        key[k] = (bits & ~7u) | (uint32_t)k;
        low |= (bits & 7u) << (3 * k);
        neg |= (v[k] < 0.f ? 1u : 0u) << k;
        S = k == 0 ? a[0] : S + a[k];
    }
    // ascending sort (Knuth's 19-comparator network for 8 inputs)
    constexpr int kNet[19][2] = {{0, 2}, {1, 3}, {4, 6}, {5, 7}, {0, 4}, {1, 5}, {2, 6},
                                 {3, 7}, {0, 1}, {2, 3}, {4, 5}, {6, 7}, {2, 4}, {3, 5},
                                 {1, 4}, {3, 6}, {1, 2}, {3, 4}, {5, 6}};
#pragma unroll
    for (int c = 0; c < 19; ++c) {
        const uint32_t x = key[kNet[c][0]], y = key[kNet[c][1]];
        key[kNet[c][0]] = x < y ? x : y;
        key[kNet[c][1]] = x < y ? y : x;
    }
    auto approx = [](uint32_t k) {
        const uint32_t b = k & ~7u;
        float f;
        __builtin_memcpy(&f, &b, 4);
        return f;
    };
    auto exact = [&](uint32_t k) {  // a of the key's coordinate
        const uint32_t i = k & 7u, b = (k & ~7u) | ((low >> (3u * i)) & 7u);
        float f;
        __builtin_memcpy(&f, &b, 4);
        return f;
    };
    const uint32_t i1 = key[7] & 7u, i2 = key[6] & 7u, i3 = key[5] & 7u;
    const uint32_t b1 = key[0] & 7u, b2 = key[1] & 7u;
    const float e1 = exact(key[7]), e2 = exact(key[6]), e3 = exact(key[5]);
    // rows +-2 at i, j: the pair's lower coordinate takes the first fma
    auto pair = [&](uint32_t p, float ap, uint32_t q, float aq, float& d) {
        const uint32_t i = p < q ? p : q, j = p < q ? q : p;
        const float ai = p < q ? ap : aq, aj = p < q ? aq : ap;
        d = __builtin_fmaf(aj, c1, __builtin_fmaf(ai, c1, 0.f));
        const uint32_t pidx = (i * (15u - i)) / 2u + (j - i - 1u);
        return 4u * pidx + (((neg >> i) & 1u) ? 0u : 2u) + (((neg >> j) & 1u) ? 0u : 1u);
    };
    float dA1, dA2;
    const uint32_t xA1 = pair(i1, e1, i2, e2, dA1);
    const uint32_t xA2 = pair(i1, e1, i3, e3, dA2);
    // rows (+-1)^8: flip sets by parity
    const bool odd = (__builtin_popcount(neg) & 1) != 0;
    const uint32_t f1 = odd ? (1u << b1) : 0u;
    const uint32_t f2 = odd ? (1u << b2) : ((1u << b1) | (1u << b2));
    auto chain = [&](uint32_t flip, float& d) {
        float acc = 0.f;
#pragma unroll
        for (int k = 0; k < 8; ++k)
            acc = __builtin_fmaf(((flip >> k) & 1u) ? -a[k] : a[k], c2, acc);
        d = acc;
        const uint32_t minus = neg ^ flip;  // coordinates with sign -
        uint32_t plus7 = 0u;                // bit 6 - k: + at coordinate k (k < 7)
#pragma unroll
        for (int k = 0; k < 7; ++k) plus7 |= (((minus >> k) & 1u) ^ 1u) << (6 - k);
        return 112u + plus7;
    };
    float dB1, dB2;
    const uint32_t xB1 = chain(f1, dB1);
    const uint32_t xB2 = chain(f2, dB2);
    // rows +-2 at i
    const uint32_t xC1 = 240u + 2u * i1 + (((neg >> i1) & 1u) ? 0u : 1u);
    const uint32_t xC2 = 240u + 2u * i2 + (((neg >> i2) & 1u) ? 0u : 1u);
    float best = dA1;
    uint32_t bi = xA1;
    auto take = [&](float d, uint32_t x) {
        if (d > best || (d == best && x < bi)) {
            best = d;
            bi = x;
        }
    };
    take(dA2, xA2);
    take(dB1, xB1);
    take(dB2, xB2);
    take(e1, xC1);
    take(e2, xC2);
    // bound on every other row
    const float m1 = approx(key[7]), m2 = approx(key[6]), m3 = approx(key[5]),
                m4 = approx(key[4]);
    const float s1 = approx(key[0]), s3 = approx(key[2]);
    const float pa = m2 + m3, pb = m1 + m4;
    const float nA = c1 * (pa > pb ? pa : pb);
    const float nB = c2 * (odd ? S - 2.f * s3 : S - 2.f * (s1 + s3));
    float bound = nA > nB ? nA : nB;
    bound = bound > m3 ? bound : m3;
    if (best > bound + 0x1p-12f * (1.f + S)) return bi;
    return root_code_full(v);
}

// 1-bit value words and v_perm_b32 selectors: per scale group the weights +-s and +-rnd(2s)
// in the activation dtype, S0 = s | rnd(2s) << 16, S1 = -s | -rnd(2s) << 16; a 256-entry
// table (4 KB) maps a code to the four selector words of its 8 weights.
constexpr int kSel1Entries = 256;

struct alignas(16) Sel1Tab {
    uint32_t w[kSel1Entries * 4];
};

constexpr Sel1Tab make_sel1_tab() {
    Sel1Tab t{};
    const RootTable r = make_root_table();
    for (int e = 0; e < kSel1Entries; ++e)
        for (int h = 0; h < 4; ++h)
            t.w[4 * e + h] = root_sel_pair(r.c[e][2 * h]) | (root_sel_pair(r.c[e][2 * h + 1]) << 16);
    return t;
}

// The selector table, built at compile time; kernels copy it into LDS (an L2 hit after the
// first workgroup) instead of deriving every entry from the code table: per entry that took
// eight byte loads and a select chain per coordinate.
static __device__ const Sel1Tab kSel1Tab = make_sel1_tab();

// Copies the table into LDS with C copies of each entry (entry stride 16 C bytes), lane l
// reading copy l % C: with C = 8 the eight lanes a b128 read serves per cycle hit distinct
// banks.  Every load of a thread is issued before its first write.  NT: threads of the
// workgroup.
template <int NT, int C = 1>
__device__ __forceinline__ void fill_sel1(uint4* tab) {
    constexpr int kItems = kSel1Entries * C;
    constexpr int kPer = (kItems + NT - 1) / NT;
    const uint4* src = reinterpret_cast<const uint4*>(kSel1Tab.w);
    uint4 v[kPer];
#pragma unroll
    for (int k = 0; k < kPer; ++k) {
        const int i = (int)threadIdx.x + k * NT;
        v[k] = src[(i < kItems ? i : 0) / C];
    }
#pragma unroll
    for (int k = 0; k < kPer; ++k) {
        const int i = (int)threadIdx.x + k * NT;
        if (i < kItems) tab[i] = v[k];
    }
}

template <int DT>
__device__ __forceinline__ uint2 values1(uint32_t s16) {
    const float s = scale_for<DT>(s16 & 0xFFFFu);
    const uint32_t a = rnd_bits<DT>(s), b = rnd_bits<DT>(2.0f * s);
    return make_uint2(a | (b << 16), (a ^ 0x8000u) | ((b ^ 0x8000u) << 16));
}

}  // namespace ojx
