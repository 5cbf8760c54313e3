// e8t_lut.h -- code -> weight expansion shared by the ternary-E8 MFMA kernels (gfx950).
//
// raw = 2*code is the base-3 number whose digits are coord+1 (lattice.py:309-318).
// raw = 81*hi + lo splits it into two 4-digit halves; each half indexes an 81-entry LDS
// table of 4 masks (8 bytes: 0xFFFF for -1, 0x0000 for 0, 0x7FFF for +1 per half-word).
// AND-ing a mask word with (s | s<<16 | 0x80008000) yields the bf16 (or fp16) pair
// coord*s exactly, since group scales are >= 0.  hi = floor(2c/81) is one mul_hi
// (exact for every valid code, checked exhaustively).  The table is "bank sliced":
// kLutSlots copies, lane l reading copy l % kLutSlots, which occupies only its own bank
// pair.  16 copies (13 KB) leave LDS for the kernels' staging buffers; 8 copies lose more
// to bank conflicts than they gain.  Kernels whose staging leaves room take 32 (LutGeom<32>:
// 2.2 instead of 3.7 clock cycles per wave-wide 8-byte read on MI355X).  The
// table is filled from a constant base table in device memory (one 8-byte load per
// thread-item), not recomputed per entry.
#pragma once

#include "e8t_device.h"

namespace ojx {

typedef __attribute__((ext_vector_type(4))) float f32x4;
typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8;
typedef __attribute__((ext_vector_type(8))) _Float16 f16x8;
typedef __attribute__((ext_vector_type(2))) uint32_t u32x2;
typedef __attribute__((ext_vector_type(3))) uint32_t u32x3;
typedef __attribute__((ext_vector_type(4))) uint32_t u32x4;


constexpr int kLutEntries = 102;            // 81 valid + slack so that any 12-bit code stays in bounds
constexpr int kLutSlots = 16;    // bank slices: lane l reads slice l % kLutSlots
static_assert(kLutSlots == 8 || kLutSlots == 16 || kLutSlots == 32, "8, 16 or 32 table slices");
constexpr uint32_t kLutStride = kLutSlots * 8;  // bytes per table entry (all slices)
// Z = 2 * code * kLutStride + slot = (code << kCodeShift) | slot; kHiMagic makes
// floor(Z * kHiMagic / 2^32) == floor(2c / 81) for every valid code c < 3281 and every slot
// offset (checked exhaustively); for invalid codes the two table addresses stay within the
// table and its zero guard entry.
constexpr int kCodeShift = kLutSlots == 32 ? 9 : (kLutSlots == 16 ? 8 : 7);
constexpr uint32_t kHiMagic = kLutSlots == 32 ? 207127u : (kLutSlots == 16 ? 414253u : 828505u);
// With 32 slices the lo address of an invalid code can fall 8 bytes below entry 0: a zero
// guard entry precedes the table.  With 8 or 16 slices every address is >= 0.
constexpr int kLutGuard = kLutSlots == 32 ? 1 : 0;
constexpr uint32_t kRsrcWord3 = 0x00020000u;  // raw buffer, 32-bit data format
// Vector offset of a buffer load that must read nothing: at or above every record count
// used here (< 2^31), so the range check returns zeros without a memory access.
constexpr uint32_t kNoRecordOffset = 0x80000000u;

// Scalar (SOFFSET) operand of a buffer instruction: the value is wave-uniform by
// construction; readfirstlane keeps it in an SGPR (the compiler otherwise may compute it
// in a VGPR and wrap the load in a waterfall loop).
__device__ __forceinline__ int uniform_offset(int64_t v) {
    return __builtin_amdgcn_readfirstlane((int)v);
}

// Table kinds.  Masks: half-word 0xFFFF for coordinate -1, 0x0000 for 0, 0x7FFF for +1
// (AND-ed with the scale word).  Values: the coordinate itself in the activation dtype
// (+-1.0 or 0), for kernels that apply the group scale to fp32 partial sums.
enum : int { kLutMasks = 0, kLutValuesBF16 = 1, kLutValuesF16 = 2 };

template <int DT>
constexpr int lut_values_kind() { return DT == kBF16 ? kLutValuesBF16 : kLutValuesF16; }

constexpr uint32_t lut_half(int kind, int d) {  // base-3 digit d = coordinate + 1
    return kind == kLutMasks ? (d == 0 ? 0xFFFFu : (d == 1 ? 0x0000u : 0x7FFFu))
         : kind == kLutValuesBF16 ? (d == 0 ? 0xBF80u : (d == 1 ? 0x0000u : 0x3F80u))
                                  : (d == 0 ? 0xBC00u : (d == 1 ? 0x0000u : 0x3C00u));
}

// Base table: word pair i + 1 holds entry i (4 digits of i, two per word, digit 0 in the
// low half-word); word pair 0 is the zero guard entry.
struct alignas(16) LutBase {
    uint32_t w[2 * (kLutEntries + 1)];
};

constexpr LutBase make_lut_base(int kind) {
    LutBase t{};
    for (int e = 0; e < kLutEntries; ++e) {
        const int d0 = e % 3, d1 = (e / 3) % 3, d2 = (e / 9) % 3, d3 = (e / 27) % 3;
        t.w[2 * (e + 1)] = lut_half(kind, d0) | (lut_half(kind, d1) << 16);
        t.w[2 * (e + 1) + 1] = lut_half(kind, d2) | (lut_half(kind, d3) << 16);
    }
    return t;
}

static __device__ const LutBase kLutBaseTab[3] = {
    make_lut_base(kLutMasks), make_lut_base(kLutValuesBF16), make_lut_base(kLutValuesF16)};

// Fills the bank-sliced table from the base table in device memory: entry e (-1 = guard),
// slice c at byte offset (e + kLutGuard) * kLutStride + c * 8 of the storage.  Each thread writes
// 16-byte items (two slices of one entry); its base-table loads are all issued before its
// first write.  NT: threads of the workgroup.
// Items (16-byte words, two slices of one entry) each thread of an NT-thread workgroup
// writes for a table of ENTRIES entries.
template <int NT, int ENTRIES, int SLOTS = kLutSlots>
struct LutFill {
    static constexpr int kGuardE = SLOTS == 32 ? 1 : 0;  // zero guard entry (32 slices)
    static constexpr int kPairs = SLOTS / 2;
    static constexpr int kItems = (ENTRIES + kGuardE) * kPairs;
    static constexpr int kPer = (kItems + NT - 1) / NT;
    uint2 v[kPer];

    // Issues this thread's base-table loads (device memory; an L2 hit after the first
    // workgroup).  Kernels issue their first weight loads between load() and store(), so
    // the two latencies overlap.
    __device__ __forceinline__ void load(int kind) {
        const uint2* tab = reinterpret_cast<const uint2*>(kLutBaseTab[kind].w);
#pragma unroll
        for (int k = 0; k < kPer; ++k) {
            const int i = (int)threadIdx.x + k * NT;
            v[k] = tab[(i < kItems ? i : 0) / kPairs + 1 - kGuardE];
        }
    }
    __device__ __forceinline__ void store(uint4* storage) const {
#pragma unroll
        for (int k = 0; k < kPer; ++k) {
            const int i = (int)threadIdx.x + k * NT;
            if (i < kItems) storage[i] = make_uint4(v[k].x, v[k].y, v[k].x, v[k].y);
        }
    }
};

// Fills the bank-sliced table from the base table in device memory: entry e (-1 = guard),
// slice c at byte offset (e + guard) * (8 * SLOTS) + c * 8 of the storage.  NT: threads
// of the workgroup.
template <int NT, int ENTRIES = kLutEntries, int SLOTS = kLutSlots>
__device__ __forceinline__ void fill_lut(uint4* storage, int kind) {
    LutFill<NT, ENTRIES, SLOTS> f;
    f.load(kind);
    f.store(storage);
}

// LDS words of the table (16-byte aligned, for the 16-byte fill writes).
constexpr int kLutStorageU4 = (kLutEntries + kLutGuard) * kLutSlots / 2;
// A table of the 81 entries that valid codes (< 3281) reach.  An invalid code then reads
// neighbouring LDS words of the same workgroup (or zeros past its allocation): a garbage
// result for garbage input, never an access outside the workgroup's LDS.
constexpr int kLutValidEntries = 81;
constexpr int kLutValidStorageU4 = (kLutValidEntries + kLutGuard) * kLutSlots / 2;
// Byte offset of entry 0 in the storage.
constexpr uint32_t kLutBaseOffset = kLutGuard * kLutStride;

// Geometry of a bank-sliced table with SLOTS copies (the constants above are SLOTS =
// kLutSlots); kernels that need another slice count than the library-wide one use these.
template <int SLOTS>
struct LutGeom {
    static_assert(SLOTS == 8 || SLOTS == 16 || SLOTS == 32, "8, 16 or 32 table slices");
    static constexpr uint32_t kStride = SLOTS * 8;
    static constexpr int kCodeShift = SLOTS == 32 ? 9 : (SLOTS == 16 ? 8 : 7);
    static constexpr uint32_t kHiMagic = SLOTS == 32 ? 207127u : (SLOTS == 16 ? 414253u : 828505u);
    static constexpr int kGuard = SLOTS == 32 ? 1 : 0;
    static constexpr int kValidStorageU4 = (81 + kGuard) * SLOTS / 2;
    static constexpr uint32_t kBaseOffset = kGuard * kStride;
};

// Z = (code_j << kCodeShift) | slot for code j (0..7) of the 12-byte, 8-code group
// (d0, d1, d2): code j occupies bits [12j, 12j+12) of the little-endian stream
// (lattice.py:375-383).
template <int J, int SHIFT = kCodeShift>
__device__ __forceinline__ uint32_t code_z(const uint32_t (&d)[3], uint32_t slot) {
    constexpr int kCodeShift = SHIFT;
    constexpr int p = 12 * J, w = p / 32, o = p % 32;
    uint32_t t;
    if constexpr (o + 12 <= 32) {
        if constexpr (o <= kCodeShift) t = d[w] << (kCodeShift - o);
        else t = d[w] >> (o - kCodeShift);
    } else {
        t = __builtin_amdgcn_alignbit(d[w + 1], d[w], o - kCodeShift);
    }
    return (t & (0xFFFu << kCodeShift)) | slot;
}

// lo address = Z - 81 * kLutStride * hi = (2c - 81 hi) * kLutStride + slot, as one
// full-rate 24-bit multiply-add (the compiler otherwise picks a 64-bit v_mad_u64_u32).
template <uint32_t STRIDE = kLutStride>
__device__ __forceinline__ uint32_t lo_addr_of(uint32_t h, uint32_t z) {
    uint32_t r;
    asm("v_mad_i32_i24 %0, %1, %2, %3" : "=v"(r) : "v"(h), "s"(-81 * (int)STRIDE), "v"(z));
    return r;
}

// Two group scales (fp16 bits, packed) -> the AND words s | s<<16 | 0x80008000 in the
// activation dtype (bf16: bf16_rne(float(s16)), lattice.py:414-418; fp16: exact).
template <int DT>
__device__ __forceinline__ void scale_words(uint32_t sc, uint32_t& w0, uint32_t& w1) {
    uint32_t p;
    if constexpr (DT == kBF16) {
        const __bf16 b0 = (__bf16)f16_bits_to_f32(sc & 0xFFFFu);  // v_cvt_pk_bf16_f32 (RNE)
        const __bf16 b1 = (__bf16)f16_bits_to_f32(sc >> 16);
        p = (uint32_t)__builtin_bit_cast(uint16_t, b0) |
            ((uint32_t)__builtin_bit_cast(uint16_t, b1) << 16);
    } else {
        p = sc;
    }
    w0 = __builtin_amdgcn_perm(p, p, 0x01000100u) | 0x80008000u;
    w1 = __builtin_amdgcn_perm(p, p, 0x03020302u) | 0x80008000u;
}

// Two group scales (fp16 bits, packed) as fp32 multipliers in the activation dtype's
// rule (bf16: bf16_rne(float(s16)), lattice.py:414-418; fp16: exact).
template <int DT>
__device__ __forceinline__ void scale_pair_f32(uint32_t sc, float& s0, float& s1) {
    const float f0 = f16_bits_to_f32(sc & 0xFFFFu), f1 = f16_bits_to_f32(sc >> 16);
    if constexpr (DT == kBF16) {
        const uint32_t p = (uint32_t)__builtin_bit_cast(uint16_t, (__bf16)f0) |
                           ((uint32_t)__builtin_bit_cast(uint16_t, (__bf16)f1) << 16);
        s0 = __uint_as_float(p << 16);
        s1 = __uint_as_float(p & 0xFFFF0000u);
    } else {
        s0 = f0;
        s1 = f1;
    }
}

template <int DT>
__device__ __forceinline__ f32x4 mfma16(const uint4& a, const uint4& b, const f32x4& c) {
    if constexpr (DT == kBF16)
        return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                       __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
    else
        return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a),
                                                      __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
}


}  // namespace ojx
