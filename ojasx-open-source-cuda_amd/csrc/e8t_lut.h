// e8t_lut.h -- code -> weight expansion shared by the ternary-E8 MFMA kernels (gfx950).
//
// raw = 2*code is the base-3 number whose digits are coord+1 (lattice.py:309-318).
// raw = 81*hi + lo splits it into two 4-digit halves; each half indexes an 81-entry LDS
// table of 4 masks (8 bytes: 0xFFFF for -1, 0x0000 for 0, 0x7FFF for +1 per half-word).
// AND-ing a mask word with (s | s<<16 | 0x80008000) yields the bf16 (or fp16) pair
// coord*s exactly, since group scales are >= 0.  hi = floor(2c/81) is one mul_hi
// (exact for every valid code, checked exhaustively).  The table is "bank sliced":
// kLutSlots copies, lane l reading copy l % kLutSlots, which occupies only its own bank
// pair -- the lanes of a ds_read_b64 phase never conflict.
#pragma once

#include "e8t_device.h"

namespace ojx {

typedef __attribute__((ext_vector_type(4))) float f32x4;
typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8;
typedef __attribute__((ext_vector_type(8))) _Float16 f16x8;
typedef __attribute__((ext_vector_type(3))) uint32_t u32x3;
typedef __attribute__((ext_vector_type(4))) uint32_t u32x4;

constexpr int kLutEntries = 102;            // 81 valid + slack so that any 12-bit code stays in bounds
constexpr int kLutSlots = 32;               // bank slices: lane l reads slice l % 32
constexpr uint32_t kLutStride = kLutSlots * 8;  // bytes per table entry (all slices)
constexpr uint32_t kHiMagic = 207127u;      // floor((512c + b) * kHiMagic / 2^32) == floor(2c / 81), b < 256
constexpr uint32_t kRsrcWord3 = 0x00020000u;  // raw buffer, 32-bit data format

// Scalar (SOFFSET) operand of a buffer instruction: the value is wave-uniform by
// construction; readfirstlane keeps it in an SGPR (the compiler otherwise may compute it
// in a VGPR and wrap the load in a waterfall loop).
__device__ __forceinline__ int uniform_offset(int64_t v) {
    return __builtin_amdgcn_readfirstlane((int)v);
}

// Mask table half-word of base-3 digit d (coord d - 1).
struct LutMasks {
    __device__ uint32_t operator()(int d) const {
        return d == 0 ? 0xFFFFu : (d == 1 ? 0x0000u : 0x7FFFu);
    }
};

// Value table half-word: coord d - 1 itself in the activation dtype (+-1.0 or 0), for
// kernels that apply the group scale to fp32 partial sums after the MFMA.
template <int DT>
struct LutValues {
    __device__ uint32_t operator()(int d) const {
        const uint32_t one = DT == kBF16 ? 0x3F80u : 0x3C00u;
        return d == 0 ? (one | 0x8000u) : (d == 1 ? 0x0000u : one);
    }
};

// Fills the bank-sliced table: entry e, slice c at byte offset (e + 1) * kLutStride + c * 8
// of the storage; entry -1 is a zero guard (with kHiMagic, the lo address of an invalid
// code >= 3281 can reach 8 bytes below entry 0; valid codes never do).
template <typename Half = LutMasks>
__device__ __forceinline__ void fill_lut(uint2* storage, Half half = Half()) {
    for (int i = threadIdx.x; i < (kLutEntries + 1) * kLutSlots; i += blockDim.x) {
        const int e = i / kLutSlots - 1;
        if (e < 0) {
            storage[i] = make_uint2(0u, 0u);
            continue;
        }
        const int d0 = e % 3, d1 = (e / 3) % 3, d2 = (e / 9) % 3, d3 = (e / 27) % 3;
        storage[i] = make_uint2(half(d0) | (half(d1) << 16), half(d2) | (half(d3) << 16));
    }
}

// Z = (code_j << 9) | slot for code j (0..7) of the 12-byte, 8-code group (d0, d1, d2):
// code j occupies bits [12j, 12j+12) of the little-endian stream (lattice.py:375-383).
template <int J>
__device__ __forceinline__ uint32_t code_z(const uint32_t (&d)[3], uint32_t slot) {
    uint32_t t;
    if constexpr (J == 0) t = d[0] << 9;
    else if constexpr (J == 1) t = d[0] >> 3;
    else if constexpr (J == 2) t = __builtin_amdgcn_alignbit(d[1], d[0], 15);
    else if constexpr (J == 3) t = d[1] << 5;
    else if constexpr (J == 4) t = d[1] >> 7;
    else if constexpr (J == 5) t = __builtin_amdgcn_alignbit(d[2], d[1], 19);
    else if constexpr (J == 6) t = d[2] << 1;
    else t = d[2] >> 11;
    return (t & 0x1FFE00u) | slot;
}

// lo address = Z - 81 * kLutStride * hi = (2c - 81 hi) * kLutStride + slot, as one
// full-rate 24-bit multiply-add (the compiler otherwise picks a 64-bit v_mad_u64_u32).
__device__ __forceinline__ uint32_t lo_addr_of(uint32_t h, uint32_t z) {
    uint32_t r;
    asm("v_mad_i32_i24 %0, %1, %2, %3" : "=v"(r) : "v"(h), "s"(-81 * (int)kLutStride), "v"(z));
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
