// e8t_gemv.hip -- decode-in-register ternary-E8 GEMV for gfx950 (batch M <= 16).
//
// y[M,N] = x[M,K] . Wq[N,K]^T (+ bias), Wq[n,k] = coord(code) * scale(n, k/32) in the
// activation dtype (bf16: coord * bf16_rne(s16), lattice.py:414-418), fp32 accumulation.
// Replaces the reference's decode-time route, which unpacks the whole layer to a dense
// bf16 matrix and then runs a dense GEMM (lattice.py:610-624); here no dense weight
// ever exists: codes stream from HBM once and are expanded in registers.
//
// Work decomposition.  A wave owns R "n-tiles" of 16 output rows and a range of
// 256-wide K chunks.  One MFMA step (v_mfma_f32_16x16x32_{bf16,f16}) contracts 32 k
// of 16 rows: lane (g = lane/16, n = lane%16) supplies the 8 weights of ONE code of
// row n -- the 8-vector that is the unit of the E8 code -- and the matching 8
// activations of x row m = lane%16.  Within a chunk, lane group g owns codes
// 8g .. 8g+7 of each row (12 contiguous bytes, one dwordx3 load per row) and the
// two group scales covering them (one dword); step j (0..7) uses code 8g+j.  The
// summation order over k is a permutation of k applied to both operands, so the
// result is the same dot product.
//
// Code -> 8 bf16 weights.  raw = 2*code is the base-3 number whose digits are
// coord+1 (lattice.py:309-318).  raw = 81*hi + lo splits it into two 4-digit
// halves, each looked up in an 81-entry LDS table of 4 masks (8 bytes: 0xFFFF for
// -1, 0x0000 for 0, 0x7FFF for +1 per half-word).  AND-ing a mask word with
// (s | s<<16 | 0x80008000) yields the bf16 (or fp16) pair coord*s exactly, since
// s >= 0.  hi = floor(2c/81) is one mul_hi (exact for every 12-bit input, checked
// exhaustively).  The table is "bank sliced": 16 copies, copy c occupying only
// bank pair c, so the 16 lanes of each ds_read_b64 phase never conflict.
//
// Grouped launches: one launch may run many independent linears (a job table in
// device memory), e.g. a decoder's q/k/v projections that share x, or a whole
// stack of layers; the workgroup grid is the concatenation of every job's grid.

#include "e8t_device.h"
#include "e8t_internal.h"

namespace ojx {

typedef __attribute__((ext_vector_type(4))) float f32x4;
typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8;
typedef __attribute__((ext_vector_type(8))) _Float16 f16x8;

constexpr int kGemvThreads = 256;           // 4 waves
constexpr int kLutEntries = 102;            // 81 valid + slack so that any 12-bit code stays in bounds
constexpr int kLutSlots = 16;               // bank slices (one per lane of a ds_read_b64 phase)
constexpr uint32_t kHiMagic = 414253u;      // floor((256c + b) * kHiMagic / 2^32) == floor(2c / 81)
constexpr int kChunk = 256;                 // K per chunk: 32 codes per row = 48 bytes

__device__ __forceinline__ uint32_t lut_mask_half(int digit) {
    return digit == 0 ? 0xFFFFu : (digit == 1 ? 0x0000u : 0x7FFFu);
}

// Fills the bank-sliced table: entry e, slot c at byte offset e*128 + c*8.
__device__ __forceinline__ void fill_lut(uint2* lut) {
    for (int i = threadIdx.x; i < kLutEntries * kLutSlots; i += blockDim.x) {
        const int e = i / kLutSlots;
        const int d0 = e % 3, d1 = (e / 3) % 3, d2 = (e / 9) % 3, d3 = (e / 27) % 3;
        lut[i] = make_uint2(lut_mask_half(d0) | (lut_mask_half(d1) << 16),
                            lut_mask_half(d2) | (lut_mask_half(d3) << 16));
    }
}

// Z = 256 * code_j + slot_byte for code j (0..7) of the 12-byte, 8-code group (d0,d1,d2):
// code j occupies bits [12j, 12j+12) of the little-endian stream (lattice.py:375-383).
template <int J>
__device__ __forceinline__ uint32_t code_z(uint32_t d0, uint32_t d1, uint32_t d2, uint32_t slot) {
    uint32_t t;
    if constexpr (J == 0) t = d0 << 8;
    else if constexpr (J == 1) t = d0 >> 4;
    else if constexpr (J == 2) t = __builtin_amdgcn_alignbit(d1, d0, 16);
    else if constexpr (J == 3) t = d1 << 4;
    else if constexpr (J == 4) t = d1 >> 8;
    else if constexpr (J == 5) t = __builtin_amdgcn_alignbit(d2, d1, 20);
    else if constexpr (J == 6) t = d2;
    else t = d2 >> 12;
    return (t & 0xFFF00u) | slot;
}

// Packs the bf16 (DT=bf16) or fp16 bits of one group scale as s | s<<16 | 0x80008000.
template <int DT>
__device__ __forceinline__ uint32_t scale_word(uint32_t s16) {
    uint32_t b;
    if constexpr (DT == kBF16) b = f32_to_bf16_bits(f16_bits_to_f32(s16));
    else b = s16;
    return (b * 0x10001u) | 0x80008000u;
}

// z - 10368 * h as one full-rate 24-bit multiply-add (the compiler otherwise picks a
// 64-bit v_mad_u64_u32 for this pattern).
__device__ __forceinline__ uint32_t mad_i24(uint32_t h, uint32_t z) {
    uint32_t r;
    asm("v_mad_i32_i24 %0, %1, %2, %3" : "=v"(r) : "v"(h), "s"(-10368), "v"(z));
    return r;
}

struct GemvLane {
    uint32_t slot;   // byte offset of this lane's bank slice
    int g;           // lane group (0..3)
    int i16;         // lane % 16
};

template <int DT>
__device__ __forceinline__ f32x4 mfma16(const uint4& a, const uint4& b, const f32x4& c) {
    if constexpr (DT == kBF16)
        return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                       __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
    else
        return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a),
                                                      __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
}

template <int DT, int R>
struct Chunk {
    uint32_t cd[R][3];   // 8 codes of each of the wave's R rows-for-this-lane
    uint32_t sc[R];      // two fp16 scales
    uint4 xa[8];         // A fragments for the 8 steps
};

// Loads are unconditional: rows past N and activation rows past M read a clamped, valid
// row; the MFMA outputs they produce are never stored.
template <int DT, int R>
__device__ __forceinline__ void load_chunk(Chunk<DT, R>& ch, int64_t c, const GemvLane& L,
                                           const uint8_t* const (&prow)[R],
                                           const uint16_t* const (&srow)[R],
                                           const uint16_t* xrow) {
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const uint32_t* p = reinterpret_cast<const uint32_t*>(prow[r] + c * 48 + 12 * L.g);
        ch.cd[r][0] = p[0];
        ch.cd[r][1] = p[1];
        ch.cd[r][2] = p[2];
        ch.sc[r] = *reinterpret_cast<const uint32_t*>(srow[r] + c * 8 + 2 * L.g);
    }
    const uint4* xp = reinterpret_cast<const uint4*>(xrow + c * kChunk + 64 * L.g);
#pragma unroll
    for (int j = 0; j < 8; ++j) ch.xa[j] = xp[j];
}

template <int DT, int R, int J>
__device__ __forceinline__ void step(const Chunk<DT, R>& ch, const uint32_t (&sw)[R][2],
                                     const char* lut, const GemvLane& L, f32x4 (&acc)[R]) {
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const uint32_t z = code_z<J>(ch.cd[r][0], ch.cd[r][1], ch.cd[r][2], L.slot);
        const uint32_t h = __umulhi(z, kHiMagic);
        const uint32_t lo_addr = mad_i24(h, z);
        const uint32_t hi_addr = h * 128u + L.slot;
        const uint2 ml = *reinterpret_cast<const uint2*>(lut + lo_addr);
        const uint2 mh = *reinterpret_cast<const uint2*>(lut + hi_addr);
        const uint32_t s = sw[r][J >> 2];
        const uint4 b = make_uint4(ml.x & s, ml.y & s, mh.x & s, mh.y & s);
        acc[r] = mfma16<DT>(ch.xa[J], b, acc[r]);
    }
}

template <int DT, int R>
__device__ __forceinline__ void compute_chunk(const Chunk<DT, R>& ch, const char* lut,
                                              const GemvLane& L, f32x4 (&acc)[R]) {
    uint32_t sw[R][2];
#pragma unroll
    for (int r = 0; r < R; ++r) {
        sw[r][0] = scale_word<DT>(ch.sc[r] & 0xFFFFu);
        sw[r][1] = scale_word<DT>(ch.sc[r] >> 16);
    }
    step<DT, R, 0>(ch, sw, lut, L, acc);
    step<DT, R, 1>(ch, sw, lut, L, acc);
    step<DT, R, 2>(ch, sw, lut, L, acc);
    step<DT, R, 3>(ch, sw, lut, L, acc);
    step<DT, R, 4>(ch, sw, lut, L, acc);
    step<DT, R, 5>(ch, sw, lut, L, acc);
    step<DT, R, 6>(ch, sw, lut, L, acc);
    step<DT, R, 7>(ch, sw, lut, L, acc);
}

__device__ __forceinline__ int find_job(const GemvJob* jobs, int njobs, int64_t wg) {
    int lo = 0, hi = njobs - 1;
    while (lo < hi) {  // last job with wg_begin <= wg
        const int mid = (lo + hi + 1) >> 1;
        if (jobs[mid].wg_begin <= wg) lo = mid;
        else hi = mid - 1;
    }
    return lo;
}

// R: n-tiles (16 rows) per wave.  S: K-split ways inside the workgroup (1, 2 or 4);
// the workgroup's 4 waves are (4/S) tile sets x S K ranges, reduced through LDS.
template <int DT, int R, int S>
__global__ __launch_bounds__(kGemvThreads) void gemv_kernel(GemvLaunch args) {
    __shared__ uint2 lut_storage[kLutEntries * kLutSlots];
    __shared__ f32x4 red[(S > 1) ? (kGemvThreads / 64) * R * 64 : 1];

    fill_lut(lut_storage);

    int64_t wg = blockIdx.x;
    GemvJob job;
    if (args.jobs != nullptr) {
        job = args.jobs[find_job(args.jobs, args.njobs, wg)];
    } else {
        job = args.inl[0];
#pragma unroll
        for (int i = 1; i < kGemvInlineJobs; ++i)
            if (i < args.njobs && wg >= args.inl[i].wg_begin) job = args.inl[i];
    }
    wg -= job.wg_begin;
    const void* xbase = job.x ? job.x : args.x;
    void* ybase = job.y ? job.y : args.y;

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int ks = wave % S;          // K range of this wave
    const int ts = wave / S;          // tile set of this wave
    GemvLane L;
    L.g = lane >> 4;
    L.i16 = lane & 15;
    L.slot = (uint32_t)L.i16 * 8u;

    const int64_t N = job.N, K = job.K;
    const int M = args.M;
    const int64_t rowbytes = K * 3 / 16;
    const int64_t srowlen = K / 32;
    const int64_t tile0 = (wg * (4 / S) + ts) * R;

    const uint8_t* prow[R];
    const uint16_t* srow[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
        int64_t row = (tile0 + r) * 16 + L.i16;
        row = row < N ? row : N - 1;
        prow[r] = job.packed + row * rowbytes;
        srow[r] = job.scales + row * srowlen;
    }
    const int xr = L.i16 < M ? L.i16 : M - 1;
    const uint16_t* xrow = reinterpret_cast<const uint16_t*>(xbase) + (int64_t)xr * K;

    const int64_t nch = K / kChunk;
    const int64_t c0 = nch * ks / S, c1 = nch * (ks + 1) / S;

    f32x4 acc[R];
#pragma unroll
    for (int r = 0; r < R; ++r) acc[r] = f32x4{0.f, 0.f, 0.f, 0.f};

    __syncthreads();  // LUT ready
    const char* lut = reinterpret_cast<const char*>(lut_storage);

    Chunk<DT, R> A, B;
    int64_t c = c0;
    if (c < c1) load_chunk<DT, R>(A, c, L, prow, srow, xrow);
    while (c + 1 < c1) {
        load_chunk<DT, R>(B, c + 1, L, prow, srow, xrow);
        compute_chunk<DT, R>(A, lut, L, acc);
        if (c + 2 < c1) load_chunk<DT, R>(A, c + 2, L, prow, srow, xrow);
        compute_chunk<DT, R>(B, lut, L, acc);
        c += 2;
    }
    if (c < c1) compute_chunk<DT, R>(A, lut, L, acc);

    if constexpr (S > 1) {
#pragma unroll
        for (int r = 0; r < R; ++r) red[(wave * R + r) * 64 + lane] = acc[r];
        __syncthreads();
        if (ks != 0) return;
#pragma unroll
        for (int r = 0; r < R; ++r) {
#pragma unroll
            for (int k2 = 1; k2 < S; ++k2) {
                const f32x4 o = red[((wave + k2) * R + r) * 64 + lane];
                acc[r] += o;
            }
        }
    }

    // lane (g, n) holds rows m = 4g + q of column n (MFMA 16x16 output layout)
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const int64_t row = (tile0 + r) * 16 + L.i16;
        if (row >= N) continue;
        const float bv = job.bias ? load_as_f32<DT>(job.bias, row) : 0.f;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const int m = 4 * L.g + q;
            if (m < M) store_from_f32<DT>(ybase, (int64_t)m * job.y_ld + job.y_col + row,
                                          acc[r][q] + bv);
        }
    }
}

// ------------------------------------------------------------------------- host side

bool gemv_supported(const void* x, const uint8_t* packed, const uint16_t* scales, const void* y,
                    int64_t M, int64_t K, int64_t gs, int dt) {
    if (dt != kBF16 && dt != kF16) return false;
    if (gs != 32 || M < 1 || M > 16 || K <= 0 || K % kChunk != 0) return false;
    if (((uintptr_t)x & 15u) || ((uintptr_t)packed & 3u) || ((uintptr_t)scales & 3u) ||
        ((uintptr_t)y & 1u))
        return false;
    return true;
}

void gemv_pick(int64_t total_tiles, int* R, int* S) {
    // Enough waves to fill 256 CUs (>= 4 per CU) first, then reuse of the x fragments
    // (R tiles per wave) -- larger R cuts the activation re-reads per weight byte.
    if (total_tiles >= 8192) { *R = 4; *S = 1; }
    else if (total_tiles >= 2048) { *R = 2; *S = 1; }
    else if (total_tiles >= 1024) { *R = 1; *S = 1; }
    else if (total_tiles >= 512) { *R = 1; *S = 2; }
    else { *R = 1; *S = 4; }
}

int64_t gemv_wgs_for(int64_t N, int R, int S) {
    const int64_t tiles = (N + 15) / 16;
    const int64_t per_wg = (int64_t)(4 / S) * R;
    return (tiles + per_wg - 1) / per_wg;
}

template <int DT, int R, int S>
static hipError_t launch_rs(const GemvLaunch& a, int64_t wgs, hipStream_t stream) {
    hipLaunchKernelGGL((gemv_kernel<DT, R, S>), dim3((unsigned)wgs), dim3(kGemvThreads), 0, stream,
                       a);
    return hipGetLastError();
}

template <int DT>
static hipError_t launch_dt(const GemvLaunch& a, int R, int S, int64_t wgs, hipStream_t stream) {
    if (R == 4 && S == 1) return launch_rs<DT, 4, 1>(a, wgs, stream);
    if (R == 2 && S == 1) return launch_rs<DT, 2, 1>(a, wgs, stream);
    if (R == 1 && S == 1) return launch_rs<DT, 1, 1>(a, wgs, stream);
    if (R == 1 && S == 2) return launch_rs<DT, 1, 2>(a, wgs, stream);
    if (R == 1 && S == 4) return launch_rs<DT, 1, 4>(a, wgs, stream);
    return hipErrorInvalidValue;
}

hipError_t launch_gemv(const GemvLaunch& a, int R, int S, int64_t wgs, int dt,
                       hipStream_t stream) {
    if (wgs <= 0) return hipSuccess;
    if (wgs > 0x7FFFFFFF) return hipErrorInvalidValue;
    return dt == kBF16 ? launch_dt<kBF16>(a, R, S, wgs, stream)
                       : launch_dt<kF16>(a, R, S, wgs, stream);
}

}  // namespace ojx
