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
// s >= 0.  hi = floor(2c/81) is one mul_hi (exact for every valid code, checked
// exhaustively).  The table is "bank sliced" (e8t_lut.h): lane l reads copy
// l % kLutSlots, which occupies only its own bank pair.
//
// Grouped launches: one launch may run many independent linears (a job table in
// device memory), e.g. a decoder's q/k/v projections that share x, or a whole
// stack of layers; the workgroup grid is the concatenation of every job's grid.

#include "e8t_device.h"
#include "e8t_internal.h"
#include "e8t_lut.h"
#include "e8t_root.h"

#include <utility>

namespace ojx {

constexpr int kGemvThreads = 256;           // 4 waves
constexpr int kChunk = 256;                 // K per chunk: 32 codes per row = 48 bytes

template <int R>
struct Codes {
    uint32_t cd[R][3];   // 8 codes (12 bytes) of each of this lane's R rows
    uint32_t sc[R];      // the two fp16 scales covering them
};

// Per-wave streaming state: buffer resources and lane offsets, fixed for the wave.
template <int R>
struct Stream {
    __amdgpu_buffer_rsrc_t packed, scales, x;
    uint32_t vo_code[R], vo_scale[R];
    uint32_t vo_x;
    bool x_live;         // this lane's activation row is < M
    uint32_t slot;       // byte offset of this lane's table slice
};

// Loads beyond the end of a weight buffer (rows >= N) return 0 (raw buffer bounds
// check); the outputs they feed are never stored.
template <int R>
__device__ __forceinline__ void load_codes(Codes<R>& ch, int64_t c, const Stream<R>& st) {
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const u32x3 v = __builtin_amdgcn_raw_buffer_load_b96(st.packed, st.vo_code[r],
                                                             uniform_offset(c * 48), 0);
        ch.cd[r][0] = v.x;
        ch.cd[r][1] = v.y;
        ch.cd[r][2] = v.z;
        ch.sc[r] = __builtin_amdgcn_raw_buffer_load_b32(st.scales, st.vo_scale[r],
                                                        uniform_offset(c * 16), 0);
    }
}

template <int R>
__device__ __forceinline__ void load_x(uint4& xa, int64_t c, int j, const Stream<R>& st) {
    if (st.x_live) {
        const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(st.x, st.vo_x + 16u * j,
                                                              uniform_offset(c * (kChunk * 2)), 0);
        xa = make_uint4(v.x, v.y, v.z, v.w);
    }
}

template <int R, int J>
__device__ __forceinline__ void lut_reads(const Codes<R>& ch, const char* lut, uint32_t slot,
                                          uint2 (&ml)[R], uint2 (&mh)[R]) {
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const uint32_t z = code_z<J>(ch.cd[r], slot);
        const uint32_t h = __umulhi(z, kHiMagic);
        ml[r] = *reinterpret_cast<const uint2*>(lut + lo_addr_of(h, z));
        mh[r] = *reinterpret_cast<const uint2*>(lut + (h * kLutStride + slot));
    }
}

template <int DT, int R, int J>
__device__ __forceinline__ void mfma_step(const uint2 (&ml)[R], const uint2 (&mh)[R],
                                          const uint32_t (&sw)[R][2], const uint4& xa,
                                          f32x4 (&acc)[R]) {
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const uint32_t s = sw[r][J >> 2];
        const uint4 b = make_uint4(ml[r].x & s, ml[r].y & s, mh[r].x & s, mh[r].y & s);
        acc[r] = mfma16<DT>(xa, b, acc[r]);
    }
}

// One 256-wide K chunk: 8 MFMA steps per row tile.  The table reads of step j+1 are
// issued before the MFMAs of step j; x fragment j is refilled with chunk `cn`'s
// fragment j as soon as step j has consumed it (cn < 0: no next chunk).
template <int DT, int R>
__device__ __forceinline__ void compute_chunk(const Codes<R>& ch, uint4 (&xa)[8], int64_t cn,
                                              const char* lut, const Stream<R>& st,
                                              f32x4 (&acc)[R]) {
    uint32_t sw[R][2];
#pragma unroll
    for (int r = 0; r < R; ++r) scale_words<DT>(ch.sc[r], sw[r][0], sw[r][1]);
    uint2 l0[R], h0[R], l1[R], h1[R];
    lut_reads<R, 0>(ch, lut, st.slot, l0, h0);
    lut_reads<R, 1>(ch, lut, st.slot, l1, h1);
    mfma_step<DT, R, 0>(l0, h0, sw, xa[0], acc);
    if (cn >= 0) load_x(xa[0], cn, 0, st);
    lut_reads<R, 2>(ch, lut, st.slot, l0, h0);
    mfma_step<DT, R, 1>(l1, h1, sw, xa[1], acc);
    if (cn >= 0) load_x(xa[1], cn, 1, st);
    lut_reads<R, 3>(ch, lut, st.slot, l1, h1);
    mfma_step<DT, R, 2>(l0, h0, sw, xa[2], acc);
    if (cn >= 0) load_x(xa[2], cn, 2, st);
    lut_reads<R, 4>(ch, lut, st.slot, l0, h0);
    mfma_step<DT, R, 3>(l1, h1, sw, xa[3], acc);
    if (cn >= 0) load_x(xa[3], cn, 3, st);
    lut_reads<R, 5>(ch, lut, st.slot, l1, h1);
    mfma_step<DT, R, 4>(l0, h0, sw, xa[4], acc);
    if (cn >= 0) load_x(xa[4], cn, 4, st);
    lut_reads<R, 6>(ch, lut, st.slot, l0, h0);
    mfma_step<DT, R, 5>(l1, h1, sw, xa[5], acc);
    if (cn >= 0) load_x(xa[5], cn, 5, st);
    lut_reads<R, 7>(ch, lut, st.slot, l1, h1);
    mfma_step<DT, R, 6>(l0, h0, sw, xa[6], acc);
    if (cn >= 0) load_x(xa[6], cn, 6, st);
    mfma_step<DT, R, 7>(l1, h1, sw, xa[7], acc);
    if (cn >= 0) load_x(xa[7], cn, 7, st);
}

// LoRA term of output (m, n) of a job (0 without an adapter).
template <int DT>
__device__ __forceinline__ float job_lora(const GemvJob& job, int64_t m, int64_t n) {
    if (job.lora_r <= 0) return 0.f;
    return lora_term<DT>(job.lora_u, job.lora_b, job.lora_r,
                         job.lora_ldu ? job.lora_ldu : job.lora_r, job.N, m, n);
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

// The job of workgroup `wg` of a launch (the device table, or the launch's inline jobs);
// `wg` becomes the workgroup's index within the job.  The compiler may merge the two sources
// into one copy through a generic pointer (flat loads into vector registers); with kScalar
// every word is then passed through readfirstlane, so that the pointers and sizes derived
// from the job, uniform by construction, stay in scalar registers: a buffer descriptor it
// cannot prove uniform makes it wrap every buffer load in a loop over the wave's distinct
// values (measured: grouped 2-bit stack 0.54 / 0.60 -> 0.47 / 0.52 ms at M = 1 / 4, 1-bit
// 0.48 / 0.51 -> 0.45 / 0.47; per-linear down at M = 16 14.9 -> 13.6 us).
template <bool kScalar = true>
__device__ __forceinline__ GemvJob gemv_job_of(const GemvLaunch& args, int64_t& wg) {
    GemvJob job;
    if (args.jobs != nullptr) {
        job = args.jobs[find_job(args.jobs, args.njobs, wg)];
    } else {
        job = args.inl[0];
#pragma unroll
        for (int i = 1; i < kGemvInlineJobs; ++i)
            if (i < args.njobs && wg >= args.inl[i].wg_begin) job = args.inl[i];
    }
    if constexpr (kScalar) {
        static_assert(sizeof(GemvJob) % 4 == 0, "job words");
        uint32_t words[sizeof(GemvJob) / 4];
        __builtin_memcpy(words, &job, sizeof(GemvJob));
#pragma unroll
        for (int i = 0; i < (int)(sizeof(GemvJob) / 4); ++i)
            words[i] = __builtin_amdgcn_readfirstlane(words[i]);
        __builtin_memcpy(&job, words, sizeof(GemvJob));
    }
    wg -= job.wg_begin;
    return job;
}

// R: n-tiles (16 rows) per wave.  S: K-split ways inside the workgroup (1, 2 or 4);
// the workgroup's 4 waves are (4/S) tile sets x S K ranges, reduced through LDS.
template <int DT, int R, int S>
__global__ __launch_bounds__(kGemvThreads) void gemv_kernel(GemvLaunch args) {
    __shared__ uint4 lut_storage[kLutStorageU4];
    __shared__ f32x4 red[(S > 1) ? (kGemvThreads / 64) * R * 64 : 1];

    fill_lut<kGemvThreads>(lut_storage, kLutMasks);

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
    const int g = lane >> 4;
    const int i16 = lane & 15;

    const int64_t N = job.N, K = job.K;
    const int M = args.M;
    const uint32_t rowbytes = (uint32_t)(K * 3 / 16);
    const uint32_t srowbytes = (uint32_t)(K / 16);
    const int64_t tile0 = (wg * (4 / S) + ts) * R;

    Stream<R> st;
    st.packed = __builtin_amdgcn_make_buffer_rsrc((void*)job.packed, (short)0,
                                                  (int)(N * rowbytes), kRsrcWord3);
    st.scales = __builtin_amdgcn_make_buffer_rsrc((void*)job.scales, (short)0,
                                                  (int)(N * srowbytes), kRsrcWord3);
    st.x = __builtin_amdgcn_make_buffer_rsrc((void*)xbase, (short)0, (int)(M * K * 2),
                                             kRsrcWord3);
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const uint32_t row = (uint32_t)((tile0 + r) * 16 + i16);
        st.vo_code[r] = row * rowbytes + 12u * g;
        st.vo_scale[r] = row * srowbytes + 4u * g;
    }
    st.vo_x = (uint32_t)(i16 * K * 2 + 128 * g);
    st.x_live = i16 < M;
    st.slot = (uint32_t)(lane & (kLutSlots - 1)) * 8u;

    const int64_t nch = K / kChunk;
    const int64_t c0 = nch * ks / S, c1 = nch * (ks + 1) / S;

    f32x4 acc[R];
#pragma unroll
    for (int r = 0; r < R; ++r) acc[r] = f32x4{0.f, 0.f, 0.f, 0.f};
    uint4 xa[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) xa[j] = make_uint4(0u, 0u, 0u, 0u);

    Codes<R> A, B;
    if (c0 < c1) {
        load_codes<R>(A, c0, st);
#pragma unroll
        for (int j = 0; j < 8; ++j) load_x(xa[j], c0, j, st);
    }
    __syncthreads();  // LUT ready
    const char* lut = reinterpret_cast<const char*>(lut_storage) + kLutBaseOffset;

    for (int64_t c = c0; c < c1; c += 2) {
        const bool has1 = c + 1 < c1, has2 = c + 2 < c1;
        if (has1) load_codes<R>(B, c + 1, st);
        compute_chunk<DT, R>(A, xa, has1 ? c + 1 : -1, lut, st, acc);
        if (!has1) break;
        if (has2) load_codes<R>(A, c + 2, st);
        compute_chunk<DT, R>(B, xa, has2 ? c + 2 : -1, lut, st, acc);
    }

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
        const int64_t row = (tile0 + r) * 16 + i16;
        if (row >= N) continue;
        const float bv = job.bias ? load_as_f32<DT>(job.bias, row) : 0.f;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const int m = 4 * g + q;
            if (m < M) store_from_f32<DT>(ybase, (int64_t)m * job.y_ld + job.y_col + row,
                                          acc[r][q] + bv + job_lora<DT>(job, m, row));
        }
    }
}

// ------------------------------------------------------------------------- streaming kernels
//
// Two streaming kernels cover launches with many row tiles (grouped launches, large N):
// the post-scaled kernel (M <= 4, 1024-k rounds) and the mask kernel (M <= 16, 512-k
// rounds).  In both, a wave owns R = 2 tiles of 16 rows; per round, its code bytes (and the
// mask kernel's scales) are fetched by 16-byte buffer->LDS loads in which consecutive lanes
// read consecutive pieces of whole row segments, into a per-wave LDS stage, then read back
// in the MFMA layout (lane (g, n): the codes of lane group g of row n).  Loads that cover
// whole row segments stream near the HBM ceiling on MI355X (about 6.3 TB/s measured),
// while one lane reading its own 48 bytes of each of 16 rows per load instruction -- the
// MFMA layout fetched directly -- stays near 4.5 TB/s.  The round's activations are staged
// in LDS by buffer->LDS loads issued one round ahead (padded rows: conflict-free reads);
// one workgroup barrier per round.

constexpr int kRound = 1024;                      // K per round
// Post-scaled kernel: tile groups per workgroup, one.  Measured on MI355X when the kernel
// could take several (32-layer decode stack, M = 1): 1 -> 3.7-3.8 TB/s, 2 -> 3.5, 4 -> 3.3,
// 8 -> 2.9; longer workgroups save table fills and prologue latency but leave a longer tail
// of partly idle CUs.
constexpr int kPsChunk = 1;
// Waves per workgroup of the post-scaled kernel.
constexpr int kPsWaves = 4;
// Waves per workgroup and table slices of the post-scaled kernel at 1 < M <= 4, two tiles
// per wave.
constexpr int kPsWavesM4 = 4;
constexpr int kPsSlotsM4 = 16;
// Row tiles (16 rows) per wave of the post-scaled kernel.
constexpr int kPsTiles = 2;
// Post-scaled launches at 1 < M <= 4 with fewer row tiles than this take one tile per wave
// (64-row workgroups: twice the workgroups, each activation round shared by 64 rows).
// Measured on the decoder's fused gate/up (1792 tiles, M = 4), per decode step of 32 layers:
// 86 us less than the staged-tile kernel; launches of 8016 tiles (lm_head) gain nothing and
// the 10,752-tile stack loses 10-15%, so they keep two tiles per wave.
constexpr int64_t kPsOneTileBelow = 4096;
// Table slices of the post-scaled kernel at M = 1.  Measured on MI355X (32-layer grouped
// stack, same box): 32 slices 0.361 ms against 0.400 ms with 16; at M = 4 the 32-slice
// table costs a workgroup per CU of residency and runs 0.470 against 0.441 ms.
constexpr int kPsSlotsM1 = 32;
constexpr uint32_t kXRow = kRound * 2 + 16;       // bytes per padded activation row in LDS

template <int R>
struct WideCodes {
    uint32_t cd[R][12];  // 48 bytes = 32 codes of one row
};

template <int R>
struct WideScales {
    uint32_t sc[R][4];   // the 8 group scales covering the 32 codes
    bool live;           // false: the lane group's k range is past K (its scales count as 0)
};

// LDS destination operand of a buffer->LDS load (kept out of templates: the host pass of
// a template instantiation rejects the address-space cast of a dependent expression).
__device__ __forceinline__ __attribute__((address_space(3))) void* lds_ptr(void* p) {
    return (__attribute__((address_space(3))) void*)p;
}

// Stages x[m][1024u .. 1024u + 1024) for m < M into LDS buffer `xs` (row stride kXRow):
// 2M wave-level loads of 1 KB each, spread over the workgroup's `waves` waves.
__device__ __forceinline__ void stage_x(char* xs, __amdgpu_buffer_rsrc_t x, int64_t u, int M,
                                        int64_t K, int wave, int lane, int waves) {
    for (int q = wave; q < 2 * M; q += waves) {
        const int m = q >> 1, half = q & 1;
        __builtin_amdgcn_raw_ptr_buffer_load_lds(
            x, lds_ptr(xs + m * kXRow + half * 1024), 16,
            (uint32_t)(m * K * 2 + half * 1024 + lane * 16), uniform_offset(u * kRound * 2), 0,
            0);
    }
}

// Table reads of code J of each tile's code words (NW words = 8 codes per 3 words), from a
// table of SL bank slices.
template <int R, int NW, int J, int SL = kLutSlots>
__device__ __forceinline__ void codes_lut(const uint32_t (&cd)[R][NW], const char* lut,
                                          uint32_t slot, uint2 (&ml)[R], uint2 (&mh)[R]) {
    using G = LutGeom<SL>;
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const uint32_t d[3] = {cd[r][3 * (J / 8)], cd[r][3 * (J / 8) + 1],
                               cd[r][3 * (J / 8) + 2]};
        const uint32_t z = code_z<J % 8, G::kCodeShift>(d, slot);
        const uint32_t h = __umulhi(z, G::kHiMagic);
        ml[r] = *reinterpret_cast<const uint2*>(lut + lo_addr_of<G::kStride>(h, z));
        mh[r] = *reinterpret_cast<const uint2*>(lut + (h * G::kStride + slot));
    }
}

// The same table reads, as one 4-word B operand per tile (lo words, hi words).
template <int R, int NW, int J, int SL = kLutSlots>
__device__ __forceinline__ void codes_lut4(const uint32_t (&cd)[R][NW], const char* lut,
                                           uint32_t slot, uint4 (&b)[R]) {
    uint2 ml[R], mh[R];
    codes_lut<R, NW, J, SL>(cd, lut, slot, ml, mh);
#pragma unroll
    for (int r = 0; r < R; ++r) b[r] = make_uint4(ml[r].x, ml[r].y, mh[r].x, mh[r].y);
}

// Operands (A fragment and table words) of the next kLookahead steps of a round, read
// ahead so that the table reads of a step have kLookahead steps of other work to land.
constexpr int kLookahead = 2;

template <int R>
struct Ahead {
    uint4 xa[kLookahead];
    uint4 b[kLookahead][R];   // table words of each tile: lo half, hi half
};

// Drops step J's operands and appends the fresh ones (for step J + kLookahead).
template <int R>
__device__ __forceinline__ void ahead_shift(Ahead<R>& ah, const uint4& xa_n, const uint4 (&b_n)[R],
                                            bool fresh) {
#pragma unroll
    for (int i = 0; i + 1 < kLookahead; ++i) {
        ah.xa[i] = ah.xa[i + 1];
#pragma unroll
        for (int r = 0; r < R; ++r) ah.b[i][r] = ah.b[i + 1][r];
    }
    if (fresh) {
        ah.xa[kLookahead - 1] = xa_n;
#pragma unroll
        for (int r = 0; r < R; ++r) ah.b[kLookahead - 1][r] = b_n[r];
    }
}

// Reads the operands of steps 0 .. kLookahead-1 of a round.
template <int R, int NW, int SL = kLutSlots>
__device__ __forceinline__ void ahead_fill(Ahead<R>& ah, const uint32_t (&cd)[R][NW],
                                           const char* lut, uint32_t slot, const char* xa_base) {
    ah.xa[0] = *reinterpret_cast<const uint4*>(xa_base);
    codes_lut4<R, NW, 0, SL>(cd, lut, slot, ah.b[0]);
    ah.xa[1] = *reinterpret_cast<const uint4*>(xa_base + 16);
    codes_lut4<R, NW, 1, SL>(cd, lut, slot, ah.b[1]);
}

__device__ __forceinline__ void vm_wait_all() {
    __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0), expcnt/lgkmcnt untouched (gfx9 encoding)
}

// Waits until at most n of this wave's loads are outstanding (gfx9 vmcnt encoding).
template <int n>
__device__ __forceinline__ void vm_wait_le() {
    static_assert(n >= 0 && n < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt(0x0F70 | (n & 15) | ((n >> 4) << 14));
}

__device__ __forceinline__ void lds_wait_all() {
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
}

// ------------------------------------------------------------------------- mask kernel
//
// M <= 16.  Rounds of 512 k: lane group g covers k = 512u + 128g + 8j, j = 0..15, i.e. 16
// codes (24 bytes) and 4 group scales (8 bytes) of each of its rows.  A wave's round of
// codes is 32 rows x 96 bytes = 3 KB, fetched into its stage by three 1-KB loads.  Step j
// decodes code j of every lane into 8 weights (table masks AND-ed with the group scale word)
// and runs one v_mfma_f32_16x16x32 per tile with the 16 activation rows as A.  Stage rows
// are rotated to spread the read-backs over the LDS banks: piece p (16 bytes) of code row n
// sits at position (p + n/4) mod 6.
//
// Scales go straight to registers in blocks of four rounds: a row's scales of rounds
// 4b .. 4b+3 are the 128 bytes at 128b, one 128-byte line (rows are K/16 bytes, a multiple
// of 128 when K % 2048 == 0), requested by four back-to-back 8-byte loads per tile (lane
// (g, n) takes bytes 32q + 8g .. 32q + 8g + 7 for round 4b + q).  Fetched a round at a time,
// each line was requested again in each of the next three rounds, by when L2 had often
// evicted it (about 4x the scale bytes read from HBM).

constexpr int kMRound = 512;                      // K per round of the mask kernel
constexpr int kMaskWaves = 8;        // waves per workgroup
constexpr uint32_t kMXRow = kMRound * 2 + 16;     // bytes per padded activation row in LDS
constexpr uint32_t kMStageBytes = 3072;           // codes of one round (two tiles)

__device__ __forceinline__ uint32_t mk_rot(uint32_t n) { return n >> 2; }

// Issues round u's three code loads into the wave's stage.
__device__ __forceinline__ void mk_issue(char* stg, __amdgpu_buffer_rsrc_t packed,
                                         const uint32_t* ld_code, int u) {
    const int so_c = uniform_offset((int64_t)u * 96);
#pragma unroll
    for (int i = 0; i < 3; ++i)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(packed, lds_ptr(stg + 1024 * i), 16, ld_code[i],
                                                 so_c, 0, 0);
}

// Loads scale block b (rounds 4b .. 4b+3) of R row tiles into registers: s[r][q] = the
// 8 bytes of lane group g in round 4b + q.  Scales of k past K (rounds past the last,
// K % 2048 != 0, and lane groups past K in a partial last round) do not exist: their loads
// take an out-of-range vector offset and read zeros (no memory traffic), which also
// zeroes those lane groups' weights of a partial round (their codes are the next row's).
// Every load is issued either way: a branch around some of them would make the results'
// registers wait for the loads.
template <int R>
__device__ __forceinline__ void mk_load_scales(uint32_t (&s)[R][4][2],
                                               __amdgpu_buffer_rsrc_t scales,
                                               const uint32_t (&vo_scale)[R], int b, int64_t K,
                                               int g) {
    const int so = uniform_offset((int64_t)b * 128);
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const bool live = (int64_t)(4 * b + q) * kMRound + 128 * g < K;
            const uint32_t o = live ? vo_scale[r] + 32u * q : kNoRecordOffset;
            const auto v = __builtin_amdgcn_raw_buffer_load_b64(scales, o, so, 0);
            s[r][q][0] = v[0];
            s[r][q][1] = v[1];
        }
}

// Stages x[m][512u .. 512u + 512) for m < M into `xs` (row stride kMXRow): one 1-KB load
// per activation row, spread over the workgroup's waves.
__device__ __forceinline__ void mk_stage_x(char* xs, __amdgpu_buffer_rsrc_t x, int64_t u, int M,
                                           int64_t K, int wave, int lane, int waves) {
    for (int m = wave; m < M; m += waves)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(x, lds_ptr(xs + m * kMXRow), 16,
                                                 (uint32_t)(m * K * 2 + lane * 16),
                                                 uniform_offset(u * kMRound * 2), 0, 0);
}

// Step J (0..15) of a mask-kernel round (R row tiles).
template <int DT, int R, int J>
__device__ __forceinline__ void mk_step(const uint32_t (&cd)[R][6], const uint32_t (&sc)[R][2],
                                        const char* lut, uint32_t slot, const char* xa_base,
                                        Ahead<R>& ah, uint32_t (&sw)[R][2], f32x4 (&acc)[R]) {
    if constexpr (J % 8 == 0) {
#pragma unroll
        for (int r = 0; r < R; ++r) scale_words<DT>(sc[r][J / 8], sw[r][0], sw[r][1]);
    }
    constexpr bool kFresh = J + kLookahead < 16;
    uint4 xa_n, b_n[R];
    if constexpr (kFresh) {
        xa_n = *reinterpret_cast<const uint4*>(xa_base + 16 * (J + kLookahead));
        codes_lut4<R, 6, (kFresh ? J + kLookahead : 0)>(cd, lut, slot, b_n);
    }
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const uint32_t s = sw[r][(J / 4) & 1];
        const uint4 m = ah.b[0][r];
        const uint4 b = make_uint4(m.x & s, m.y & s, m.z & s, m.w & s);
        acc[r] = mfma16<DT>(ah.xa[0], b, acc[r]);
    }
    if constexpr (J + 1 < 16) ahead_shift<R>(ah, xa_n, b_n, kFresh);
}

template <int DT, int R, int... J>
__device__ __forceinline__ void mk_steps(const uint32_t (&cd)[R][6], const uint32_t (&sc)[R][2],
                                         const char* lut, uint32_t slot, const char* xa_base,
                                         Ahead<R>& ah, uint32_t (&sw)[R][2], f32x4 (&acc)[R],
                                         std::integer_sequence<int, J...>) {
    (mk_step<DT, R, J>(cd, sc, lut, slot, xa_base, ah, sw, acc), ...);
}

// MMAX: activation rows staged (M <= MMAX); W: waves per workgroup (they share the table
// and the activation stage).  One tile group (W x 2 row tiles) per workgroup.
template <int DT, int MMAX, int W>
__global__ __launch_bounds__(64 * W) void gemv_mask_kernel(GemvLaunch args) {
    constexpr int R = 2;
    __shared__ uint4 lut_storage[kLutValidStorageU4];
    __shared__ __attribute__((aligned(16))) char xs_storage[2][MMAX * kMXRow];
    __shared__ __attribute__((aligned(16))) char stage[W][kMStageBytes];

    fill_lut<64 * W, kLutValidEntries>(lut_storage, kLutMasks);

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
    const int g = lane >> 4;
    const int i16 = lane & 15;
    const int64_t N = job.N, K = job.K;
    const int M = args.M;
    const uint32_t rowbytes = (uint32_t)(K * 3 / 16);
    const uint32_t srowbytes = (uint32_t)(K / 16);
    const int64_t tile0 = (wg * W + wave) * R;
    const uint32_t row0 = (uint32_t)(tile0 * 16);

    const __amdgpu_buffer_rsrc_t packed = __builtin_amdgcn_make_buffer_rsrc(
        (void*)job.packed, (short)0, (int)(N * rowbytes), kRsrcWord3);
    const __amdgpu_buffer_rsrc_t scales = __builtin_amdgcn_make_buffer_rsrc(
        (void*)job.scales, (short)0, (int)(N * srowbytes), kRsrcWord3);
    const __amdgpu_buffer_rsrc_t xr = __builtin_amdgcn_make_buffer_rsrc(
        (void*)xbase, (short)0, (int)(M * K * 2), kRsrcWord3);

    // stage slot s (16 bytes) of load i holds piece p of row n of tile r
    uint32_t ld_code[3];
#pragma unroll
    for (int i = 0; i < 3; ++i) {
        const uint32_t s = 64u * i + lane, r = s / 96u, w96 = s % 96u;
        const uint32_t n = w96 / 6u, pos = w96 % 6u;
        const uint32_t p = (pos + 6u - mk_rot(n)) % 6u;
        ld_code[i] = (row0 + 16u * r + n) * rowbytes + 16u * p;
    }
    uint32_t vo_scale[R];
#pragma unroll
    for (int r = 0; r < R; ++r) vo_scale[r] = (row0 + 16u * r + i16) * srowbytes + 8u * g;
    // read-back offsets of this lane's 8-byte words (codes: words 3g .. 3g+2 of its row)
    uint32_t rd_code[3];
#pragma unroll
    for (int t = 0; t < 3; ++t) {
        const uint32_t wd = 3u * g + t, p = wd >> 1;
        rd_code[t] = 96u * i16 + 16u * ((p + mk_rot(i16)) % 6u) + 8u * (wd & 1u);
    }
    const uint32_t slot = (uint32_t)(lane & (kLutSlots - 1)) * 8u;
    const int mrow = i16 < M ? i16 : M - 1;
    const uint32_t xa_off = (uint32_t)(mrow * kMXRow + 256 * g);

    const int T = (int)((K + kMRound - 1) / kMRound);
    f32x4 acc[R];
#pragma unroll
    for (int r = 0; r < R; ++r) acc[r] = f32x4{0.f, 0.f, 0.f, 0.f};

    char* const stg = stage[wave];
    uint32_t scb[R][4][2];
    mk_issue(stg, packed, ld_code, 0);
    mk_load_scales<R>(scb, scales, vo_scale, 0, K, g);
    mk_stage_x(xs_storage[0], xr, 0, M, K, wave, lane, W);
    vm_wait_all();
    __syncthreads();  // table, round-0 weights and activations ready
    const char* lut = reinterpret_cast<const char*>(lut_storage) + kLutBaseOffset;

    // Round u = 4 v + Q (rounds unrolled by four, so that the scale block entry and the
    // activation buffer of each round are compile-time choices); false after the last round.
    auto round = [&](int u, auto qc) -> bool {
        constexpr int Q = decltype(qc)::value;
        uint32_t cd[R][6], sc[R][2];
#pragma unroll
        for (int r = 0; r < R; ++r) {
#pragma unroll
            for (int t = 0; t < 3; ++t) {
                const uint2 v = *reinterpret_cast<const uint2*>(stg + 1536 * r + rd_code[t]);
                cd[r][2 * t] = v.x;
                cd[r][2 * t + 1] = v.y;
            }
            // zero for lane groups past K in a partial last round (mk_load_scales), whose
            // codes are the next row's
            sc[r][0] = scb[r][Q][0];
            sc[r][1] = scb[r][Q][1];
        }
        lds_wait_all();  // the read-back has landed: the stage may be refilled
        const bool has = u + 1 < T;  // uniform over the workgroup
        if (has) {
            mk_issue(stg, packed, ld_code, u + 1);
            mk_stage_x(xs_storage[(Q + 1) & 1], xr, u + 1, M, K, wave, lane, W);
            // the block's last round has taken its scales: fetch the next block
            if constexpr (Q == 3) mk_load_scales<R>(scb, scales, vo_scale, (u + 1) >> 2, K, g);
        }
        const char* xa_base = xs_storage[Q & 1] + xa_off;
        Ahead<R> ah;
        uint32_t sw[R][2];
        ahead_fill<R, 6>(ah, cd, lut, slot, xa_base);
        mk_steps<DT, 2>(cd, sc, lut, slot, xa_base, ah, sw, acc,
                        std::make_integer_sequence<int, 16>{});
        if (!has) return false;
        vm_wait_all();
        __syncthreads();  // next round's stage (own) and activations (shared) ready
        return true;
    };
    for (int u = 0;; u += 4) {
        if (!round(u, std::integral_constant<int, 0>{})) break;
        if (!round(u + 1, std::integral_constant<int, 1>{})) break;
        if (!round(u + 2, std::integral_constant<int, 2>{})) break;
        if (!round(u + 3, std::integral_constant<int, 3>{})) break;
    }

    // lane (g, n) holds rows m = 4g + q of column n (MFMA 16x16 output layout)
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const int64_t row = (tile0 + r) * 16 + i16;
        if (row >= N) continue;
        const float bv = job.bias ? load_as_f32<DT>(job.bias, row) : 0.f;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const int m = 4 * g + q;
            if (m < M) store_from_f32<DT>(ybase, (int64_t)m * job.y_ld + job.y_col + row,
                                          acc[r][q] + bv + job_lora<DT>(job, m, row));
        }
    }
}

// ------------------------------------------------------------------------- post-scaled kernel
//
// Streaming kernel for M <= 4 (token-by-token decode).  Same rounds as the wide kernel, but
// the table holds the coordinates themselves (+-1, 0 in the activation dtype) and the group
// scale multiplies fp32 partial sums instead of every decoded weight:
//
//   A row a = 4*g' + m carries activation row m, but only in the k slots of lane group
//   g' (lanes whose A row does not match their lane group read a zero block), so
//   D[4g' + m][n] = sum over lane group g''s 8 k of one step = the contribution of ONE
//   scale group (lane group g' at step j covers k = 1024u + 256g' + 8j, group 8g' + j/4).
//   In the MFMA output layout lane (g', n) holds D rows 4g' + q, i.e. exactly the partials
//   of its own codes for activation rows q = 0..3.  Four steps (one scale group) accumulate
//   into D; then acc[q] += s(n, group) * D[q], with the scale this lane already holds.
//
// The sum over the four lane groups of a row is formed once, at the end.  Per code this
// removes the four mask ANDs and the scale-word packing of the wide kernel; the weights are
// still coord * scale in the activation dtype's rule (bf16: bf16_rne(s16)), applied in fp32.
//
// Weight stream.  In round u the R row tiles of a wave need 16R rows x 192 bytes of codes
// (bytes 192u .. 192u+191 of each row: 128 codes) and 16R rows x 64 bytes of scales.  They
// are fetched by 16-byte buffer->LDS loads in which the 64 lanes of a load read consecutive
// 16-byte pieces of whole row segments -- each load covers complete 192-byte (64-byte) runs,
// the pattern that streams at the HBM ceiling -- into a per-wave LDS stage.  At the start of
// the round every lane reads back its own blocks in the MFMA layout: lane (g, n) takes the
// 48 code bytes 48g .. 48g+47 (codes 32g .. 32g+31) and the 16 scale bytes 16g .. 16g+15 of
// row n of each tile.  Within a row the four lane-group blocks are rotated: block g sits at
// position (g + tau(n)) mod 4, tau(n) = (n + n/4) mod 4, so the read-backs of the 16 rows
// hit distinct LDS banks.  The next round's loads are issued right after the read-back and
// have the whole round's compute to land.

__device__ __forceinline__ uint32_t ps_tau(uint32_t n) { return (n + (n >> 2)) & 3u; }

// One round of one wave's codes, in LDS.
template <int R>
struct PsStage {
    uint4 codes[3 * R][64];   // tile r row n block position q piece t: slot 192r + 12n + 3q + t
};

template <int R>
struct PsStream {
    __amdgpu_buffer_rsrc_t packed, scales, x;
    uint32_t ld_code[3 * R];  // byte offset of the code piece this lane fetches per load
    uint32_t vo_scale[R];     // byte offset of this lane's 8 scales (tile group c0, round 0)
    uint32_t rd_code;         // byte offset of this lane's code block in a stage tile
};


// Issues the code loads of round u of the tile group whose rows start `code_shift` bytes
// after tile group c0's into the stage at `stg` (a PsStage of `tiles` tiles).  Loads past
// the buffer's end read zeros.  (Not a template: the host pass rejects this builtin inside
// a function template instantiated from a kernel template.)
__device__ __forceinline__ void ps_issue(char* stg, __amdgpu_buffer_rsrc_t packed,
                                         const uint32_t* ld_code, int tiles, int64_t code_shift,
                                         int u) {
    const int so = uniform_offset(code_shift + (int64_t)u * 192);
#pragma unroll
    for (int i = 0; i < 3 * tiles; ++i)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(packed, lds_ptr(stg + 1024 * i), 16, ld_code[i],
                                                 so, 0, 0);
}

// The 8 scales of this lane's codes in round u (16 contiguous bytes per lane: every load
// covers whole 64-byte row segments).  Lane groups past K in a partial last round read the
// next row's codes: sc.live is false and their scales count as zero where they are used,
// so those codes contribute exactly zero.  (Zeroing the loaded words here would make the
// compiler wait for the load, and with it for every load issued before it, right away.)
template <int R>
__device__ __forceinline__ void ps_load_scales(WideScales<R>& sc, const PsStream<R>& st,
                                               int64_t scale_shift, int u, int64_t K, int g) {
    const bool live = (int64_t)u * kRound + 256 * g < K;
    const int so = uniform_offset(scale_shift + (int64_t)u * 64);
    sc.live = live;
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(st.scales, st.vo_scale[r], so, 0);
        sc.sc[r][0] = v.x;
        sc.sc[r][1] = v.y;
        sc.sc[r][2] = v.z;
        sc.sc[r][3] = v.w;
    }
}

// The scales of rounds u and u + 1 (u even): a row's 128 scale bytes of the pair are one
// 128-byte line (rows are K/16 bytes, a multiple of 128 when K % 2048 == 0), requested by
// two back-to-back loads per tile instead of one half a round apart, by when L2 may have
// evicted the line.  A pair whose second round does not exist (odd round count) points
// that load at an out-of-range vector offset: it reads nothing (zeros, no memory traffic),
// and s1 is then never used.
template <int R>
__device__ __forceinline__ void ps_load_scale_pair(WideScales<R>& s0, WideScales<R>& s1,
                                                   const PsStream<R>& st, int64_t scale_shift,
                                                   int u, int64_t K, int g) {
    s0.live = (int64_t)u * kRound + 256 * g < K;
    s1.live = (int64_t)(u + 1) * kRound + 256 * g < K;
    const bool second = (int64_t)(u + 1) * kRound < K;  // wave-uniform
    const int so = uniform_offset(scale_shift + (int64_t)u * 64);
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const u32x4 v0 = __builtin_amdgcn_raw_buffer_load_b128(st.scales, st.vo_scale[r], so, 0);
        const u32x4 v1 = __builtin_amdgcn_raw_buffer_load_b128(
            st.scales, second ? st.vo_scale[r] + 64u : kNoRecordOffset, so, 0);
        s0.sc[r][0] = v0.x;
        s0.sc[r][1] = v0.y;
        s0.sc[r][2] = v0.z;
        s0.sc[r][3] = v0.w;
        s1.sc[r][0] = v1.x;
        s1.sc[r][1] = v1.y;
        s1.sc[r][2] = v1.z;
        s1.sc[r][3] = v1.w;
    }
}

// This lane's codes of the staged round (MFMA layout).
template <int R>
__device__ __forceinline__ void ps_readback(const PsStage<R>& stg, const PsStream<R>& st,
                                            WideCodes<R>& w) {
    const char* cb = reinterpret_cast<const char*>(&stg.codes[0][0]) + st.rd_code;
#pragma unroll
    for (int r = 0; r < R; ++r) {
#pragma unroll
        for (int t = 0; t < 3; ++t) {
            const uint4 v = *reinterpret_cast<const uint4*>(cb + 3072 * r + 16 * t);
            w.cd[r][4 * t + 0] = v.x;
            w.cd[r][4 * t + 1] = v.y;
            w.cd[r][4 * t + 2] = v.z;
            w.cd[r][4 * t + 3] = v.w;
        }
    }
}

// Keeps all four result registers of an MFMA allocated up to this point.  With M == 1 only
// result 0 is read; the compiler would otherwise hand the other three registers to VALU
// code right after the MFMA issues, while the MFMA may still write them back (observed:
// corrupted code registers and wrong outputs on gfx950).  The empty asm takes the
// post-scale FMA's result as well, so it sits after the FMA that reads the MFMA result:
// by then the write-back has landed and the registers may be reused.
__device__ __forceinline__ void keep_mfma_result(const f32x4& d, float& consumer) {
    asm volatile("" : "+v"(consumer) : "v"(d));
}

// Step J of a post-scaled round; d[r] accumulates the current scale group of tile r.  SL:
// bank slices of the table.
template <int DT, int R, int MM, int J, int SL>
__device__ __forceinline__ void ps_step(const WideCodes<R>& w, const WideScales<R>& sc,
                                        const char* lut, uint32_t slot, const char* xa_base,
                                        Ahead<R>& ah, float (&sf)[R][2], f32x4 (&d)[R],
                                        float (&acc)[R][MM]) {
    if constexpr (J % 4 == 0 && J > 0) {
        // scale group J/4 - 1 is complete in d
#pragma unroll
        for (int r = 0; r < R; ++r) {
#pragma unroll
            for (int q = 0; q < MM; ++q)
                acc[r][q] = __builtin_fmaf(d[r][q], sf[r][(J / 4 - 1) & 1], acc[r][q]);
            keep_mfma_result(d[r], acc[r][0]);
        }
    }
    if constexpr (J % 8 == 0) {
#pragma unroll
        for (int r = 0; r < R; ++r)
            scale_pair_f32<DT>(sc.live ? sc.sc[r][J / 8] : 0u, sf[r][0], sf[r][1]);
    }
    constexpr bool kFresh = J + kLookahead < 32;
    uint4 xa_n, b_n[R];
    if constexpr (kFresh) {
        xa_n = *reinterpret_cast<const uint4*>(xa_base + 16 * (J + kLookahead));
        codes_lut4<R, 12, (kFresh ? J + kLookahead : 0), SL>(w.cd, lut, slot, b_n);
    }
#pragma unroll
    for (int r = 0; r < R; ++r)
        d[r] = mfma16<DT>(ah.xa[0], ah.b[0][r], J % 4 == 0 ? f32x4{0.f, 0.f, 0.f, 0.f} : d[r]);
    if constexpr (J + 1 < 32) ahead_shift<R>(ah, xa_n, b_n, kFresh);
    if constexpr (J == 31) {
#pragma unroll
        for (int r = 0; r < R; ++r) {
#pragma unroll
            for (int q = 0; q < MM; ++q)
                acc[r][q] = __builtin_fmaf(d[r][q], sf[r][1], acc[r][q]);
            keep_mfma_result(d[r], acc[r][0]);
        }
    }
}

template <int DT, int R, int MM, int SL, int... J>
__device__ __forceinline__ void ps_steps(const WideCodes<R>& w, const WideScales<R>& sc,
                                         const char* lut, uint32_t slot, const char* xa_base,
                                         Ahead<R>& ah, float (&sf)[R][2], f32x4 (&d)[R],
                                         float (&acc)[R][MM], std::integer_sequence<int, J...>) {
    (ps_step<DT, R, MM, J, SL>(w, sc, lut, slot, xa_base, ah, sf, d, acc), ...);
}

template <int DT, int R, int MM, int SL = kLutSlots>
__device__ __forceinline__ void ps_round(const WideCodes<R>& w, const WideScales<R>& sc,
                                         const char* lut, uint32_t slot, const char* xa_base,
                                         float (&acc)[R][MM]) {
    Ahead<R> ah;
    float sf[R][2];
    f32x4 d[R];
    ahead_fill<R, 12, SL>(ah, w.cd, lut, slot, xa_base);
    ps_steps<DT, R, MM, SL>(w, sc, lut, slot, xa_base, ah, sf, d, acc,
                            std::make_integer_sequence<int, 32>{});
}

// Bias bits of this lane's rows of one tile group (0 without bias; rows past N read row
// N - 1 and are never stored).  Unconditional loads whose conversion waits until the
// store, so that issuing them costs no wait.
template <int DT, int R>
__device__ __forceinline__ void ps_load_bias(const GemvJob& job, int64_t tile0, int lane,
                                             uint32_t (&bv)[R]) {
    const int i16 = lane & 15;
#pragma unroll
    for (int r = 0; r < R; ++r) bv[r] = 0u;
    if (!job.bias) return;
#pragma unroll
    for (int r = 0; r < R; ++r) {
        int64_t row = (tile0 + r) * 16 + i16;
        row = row < job.N ? row : job.N - 1;
        // global (not flat) loads: a wait for a flat load is a wait for every load
        if constexpr (DT == kF32)
            bv[r] = ((const __attribute__((address_space(1))) uint32_t*)job.bias)[row];
        else
            bv[r] = ((const __attribute__((address_space(1))) uint16_t*)job.bias)[row];
    }
}

template <int DT> __device__ __forceinline__ float bias_bits_to_f32(uint32_t b) {
    if constexpr (DT == kF32) return __uint_as_float(b);
    else if constexpr (DT == kF16) return f16_bits_to_f32(b);
    else return bf16_bits_to_f32(b);
}

// Sums the four lane groups of each row and stores one tile group's outputs (lane group q
// stores activation row q) with the bias values bv (ps_load_bias, loaded before the next
// item's prefetch so that waiting for them does not wait for the prefetch); clears the
// accumulators.
template <int DT, int R, int MM>
__device__ __forceinline__ void ps_store(const GemvJob& job, void* ybase, int M, int64_t tile0,
                                         int lane, float (&acc)[R][MM], const uint32_t (&bv)[R]) {
    const int g = lane >> 4, i16 = lane & 15;
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const int64_t row = (tile0 + r) * 16 + i16;
        float out = 0.f;
#pragma unroll
        for (int q = 0; q < MM; ++q) {
            float v = acc[r][q];
            v += __shfl_xor(v, 16);
            v += __shfl_xor(v, 32);
            if (q == g) out = v;
            acc[r][q] = 0.f;
        }
        if (row < job.N && g < M)
            store_from_f32<DT>(ybase, (int64_t)g * job.y_ld + job.y_col + row,
                               out + bias_bits_to_f32<DT>(bv[r]) + job_lora<DT>(job, g, row));
    }
}

// MM: activation rows handled (1 or 4; M <= MM); W: waves per workgroup.  A workgroup
// runs one tile group (W * R row tiles) of one job: its items are the tile group's rounds,
// so the round of each item of the loop (unrolled by two) has a compile-time parity.
// (Several tile groups per workgroup, one pipeline across them, measured slower: see
// kPsChunk.)
template <int DT, int R, int MM, int W>
__global__ __launch_bounds__(64 * W) void gemv_ps_kernel(GemvLaunch args) {
    static_assert(MM == 1 || MM == 4, "post-scaled layout holds at most 4 activation rows");
    static_assert(kPsChunk == 1, "one tile group per workgroup: its items are its rounds");
    // Table slices: 32 at M = 1 (conflict-free 8-byte reads; the 20 KB table still leaves
    // three workgroups per CU), 16 at M <= 4, whose larger activation buffers need the LDS.
    constexpr int SL = MM == 1 ? kPsSlotsM1 : (R == kPsTiles ? kPsSlotsM4 : kLutSlots);
    using G = LutGeom<SL>;
    __shared__ uint4 lut_storage[G::kValidStorageU4];
    // Two activation buffers, separate LDS objects, each ending in 512 zero bytes (the A rows
    // outside a lane's group): every activation read then points into one known buffer, so
    // the compiler does not hold it behind the pending buffer->LDS loads into the other one
    // (or into the code stage).
    constexpr int kXBytes = MM * kXRow;
    __shared__ __attribute__((aligned(16))) char xsa[kXBytes + 512];
    __shared__ __attribute__((aligned(16))) char xsb[kXBytes + 512];
    __shared__ PsStage<R> stage[W];

    fill_lut<64 * W, kLutValidEntries, SL>(lut_storage, lut_values_kind<DT>());
    if (threadIdx.x < 32) {
        reinterpret_cast<uint4*>(xsa + kXBytes)[threadIdx.x] = make_uint4(0u, 0u, 0u, 0u);
        reinterpret_cast<uint4*>(xsb + kXBytes)[threadIdx.x] = make_uint4(0u, 0u, 0u, 0u);
    }

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
    const int g = lane >> 4;
    const int i16 = lane & 15;
    const int64_t N = job.N, K = job.K;
    const int M = args.M;
    const uint32_t rowbytes = (uint32_t)(K * 3 / 16);
    const uint32_t srowbytes = (uint32_t)(K / 16);
    const int64_t tile0 = (wg * W + wave) * R;  // this wave's first row tile

    PsStream<R> st;
    st.packed = __builtin_amdgcn_make_buffer_rsrc((void*)job.packed, (short)0,
                                                  (int)(N * rowbytes), kRsrcWord3);
    st.scales = __builtin_amdgcn_make_buffer_rsrc((void*)job.scales, (short)0,
                                                  (int)(N * srowbytes), kRsrcWord3);
    st.x = __builtin_amdgcn_make_buffer_rsrc((void*)xbase, (short)0, (int)(M * K * 2),
                                             kRsrcWord3);
    const uint32_t row0 = (uint32_t)(tile0 * 16);
#pragma unroll
    for (int i = 0; i < 3 * R; ++i) {
        // stage slot s = 64 i + lane: tile s / 192, row n, block position q, piece t
        const uint32_t s = 64u * i + lane, r = s / 192u, w192 = s % 192u;
        const uint32_t n = w192 / 12u, pos = w192 % 12u, q = pos / 3u, t = pos % 3u;
        const uint32_t gg = (q - ps_tau(n)) & 3u;
        st.ld_code[i] = (row0 + 16u * r + n) * rowbytes + 16u * (3u * gg + t);
    }
#pragma unroll
    for (int r = 0; r < R; ++r) st.vo_scale[r] = (row0 + 16u * r + i16) * srowbytes + 16u * g;
    const uint32_t q_me = ((uint32_t)g + ps_tau((uint32_t)i16)) & 3u;
    st.rd_code = (12u * i16 + 3u * q_me) * 16u;
    const uint32_t slot = (uint32_t)(lane & (SL - 1)) * 8u;

    // A row i16 = 4 g' + m: live in lane group g' only, for activation rows m < M
    const int am = i16 & 3;
    const bool a_live = (i16 >> 2) == g && am < M;
    const char* xa0 = xsa + (a_live ? am * kXRow + 512 * g : kXBytes);
    const char* xa1 = xsb + (a_live ? am * kXRow + 512 * g : kXBytes);

    // Items are the rounds u; item u is processed while round u + 1's codes, scales and
    // activations are fetched.  Items alternate between the activation buffers xsa and xsb
    // (the loop is unrolled by two so that each buffer is a compile-time choice).
    const int T = (int)((K + kRound - 1) / kRound);
    float acc[R][MM];
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
        for (int q = 0; q < MM; ++q) acc[r][q] = 0.f;

    const PsStage<R>& stg = stage[wave];
    char* const stg_bytes = reinterpret_cast<char*>(&stage[wave]);
    WideCodes<R> w;
    WideScales<R> sc, sc_next, sc_odd;  // sc_odd: the odd round of the current scale pair
    ps_issue(stg_bytes, st.packed, st.ld_code, R, 0, 0);
    ps_load_scale_pair<R>(sc, sc_odd, st, 0, 0, K, g);
    stage_x(xsa, st.x, 0, M, K, wave, lane, W);
    vm_wait_all();
    __syncthreads();  // table, zero blocks, round-0 weights and activations ready
    const char* lut = reinterpret_cast<const char*>(lut_storage) + G::kBaseOffset;

    int u = 0;
    // one item (round u, parity P = u % 2): computes from the activation buffer behind
    // xa_cur, fetches round u + 1 into xs_next; false after the last round.  An odd item
    // fetches the next scale pair, an even one takes the odd half of its own.
    auto item = [&](const char* xa_cur, char* xs_next, auto pc) -> bool {
        constexpr int P = decltype(pc)::value;
        ps_readback<R>(stg, st, w);
        uint32_t bv[R];
        if (u == T - 1) ps_load_bias<DT, R>(job, tile0, lane, bv);
        lds_wait_all();  // the read-back has landed: the stage may be refilled
        const bool has = u + 1 < T;  // uniform over the workgroup
        if (has) {
            ps_issue(stg_bytes, st.packed, st.ld_code, R, 0, u + 1);
            if constexpr (P == 1)
                ps_load_scale_pair<R>(sc_next, sc_odd, st, 0, u + 1, K, g);
            else
                sc_next = sc_odd;
            stage_x(xs_next, st.x, u + 1, M, K, wave, lane, W);
        }
        ps_round<DT, R, MM, SL>(w, sc, lut, slot, xa_cur, acc);
        if (u == T - 1) ps_store<DT, R, MM>(job, ybase, M, tile0, lane, acc, bv);
        if (!has) return false;
        vm_wait_all();
        __syncthreads();  // next item's codes (own stage) and activations (shared) ready
        sc = sc_next;
        ++u;
        return true;
    };
    for (;;) {
        if (!item(xa0, xsb, std::integral_constant<int, 0>{})) break;
        if (!item(xa1, xsa, std::integral_constant<int, 1>{})) break;
    }
}

// ------------------------------------------------------------------------- small-layer kernel
//
// Post-scaled kernel for launches with few row tiles and M <= 4 (per-linear decode of
// q/k/v/o/down-sized layers): one 16-row tile per workgroup, whose W waves take the 1024-k
// rounds u = w, w + W, ... of that tile.  Each wave stages its own round's codes (coalesced,
// as above) and activations in LDS and waits only for its own loads; the waves' partial sums
// are added through LDS at the end.  A layer's weights are thus requested almost at once:
// a q/o-sized layer (256 tiles) occupies 256 workgroups for about one memory round trip,
// instead of a chain of dependent activation loads per chunk.

// Waves per workgroup at M <= 4 (the rounds of a tile spread over more waves: the kernel's
// main customer, the down projection at M = 4, K = 14336, runs 14 rounds per tile; with one
// workgroup per CU, 4 waves leave one wave per SIMD to run 3-4 rounds back to back).
// Measured on MI355X (same box): 4 waves 12.0 us, 8 waves 9.7 us; a second activation
// buffer per wave (double buffering) instead: 11.9 us.
constexpr int kPskWavesM4 = 8;

template <int DT, int MM, int W>
__global__ __launch_bounds__(64 * W) void gemv_psk_kernel(GemvLaunch args) {
    static_assert(MM == 1 || MM == 4, "post-scaled layout holds at most 4 activation rows");
    constexpr int R = 1;
    __shared__ uint4 lut_storage[kLutValidStorageU4];
    __shared__ __attribute__((aligned(16))) char stage[W][3072];
    __shared__ __attribute__((aligned(16))) char xs[W][MM * kXRow];
    __shared__ __attribute__((aligned(16))) uint4 xzero[32];
    __shared__ float red[W][MM][64];

    fill_lut<64 * W, kLutValidEntries>(lut_storage, lut_values_kind<DT>());
    if (threadIdx.x < 32) xzero[threadIdx.x] = make_uint4(0u, 0u, 0u, 0u);

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
    const int g = lane >> 4;
    const int i16 = lane & 15;
    const int64_t N = job.N, K = job.K;
    const int M = args.M;
    const uint32_t rowbytes = (uint32_t)(K * 3 / 16);
    const uint32_t srowbytes = (uint32_t)(K / 16);
    const int64_t tile0 = wg;
    const uint32_t row0 = (uint32_t)(tile0 * 16);

    PsStream<R> st;
    st.packed = __builtin_amdgcn_make_buffer_rsrc((void*)job.packed, (short)0,
                                                  (int)(N * rowbytes), kRsrcWord3);
    st.scales = __builtin_amdgcn_make_buffer_rsrc((void*)job.scales, (short)0,
                                                  (int)(N * srowbytes), kRsrcWord3);
    st.x = __builtin_amdgcn_make_buffer_rsrc((void*)xbase, (short)0, (int)(M * K * 2),
                                             kRsrcWord3);
#pragma unroll
    for (int i = 0; i < 3; ++i) {
        const uint32_t s = 64u * i + lane;  // stage slot: row n, block position q, piece t
        const uint32_t n = s / 12u, pos = s % 12u, q = pos / 3u, t = pos % 3u;
        const uint32_t gg = (q - ps_tau(n)) & 3u;
        st.ld_code[i] = (row0 + n) * rowbytes + 16u * (3u * gg + t);
    }
    st.vo_scale[0] = (row0 + i16) * srowbytes + 16u * g;
    const uint32_t q_me = ((uint32_t)g + ps_tau((uint32_t)i16)) & 3u;
    st.rd_code = (12u * i16 + 3u * q_me) * 16u;
    const uint32_t slot = (uint32_t)(lane & (kLutSlots - 1)) * 8u;

    // A row i16 = 4 g' + m: live in lane group g' only, for activation rows m < M
    const int am = i16 & 3;
    const bool a_live = (i16 >> 2) == g && am < M;
    const char* xa = a_live ? xs[wave] + am * kXRow + 512 * g
                            : reinterpret_cast<const char*>(xzero);

    const int T = (int)((K + kRound - 1) / kRound);
    float acc[R][MM];
#pragma unroll
    for (int q = 0; q < MM; ++q) acc[0][q] = 0.f;

    __syncthreads();  // table and zero block ready
    const char* lut = reinterpret_cast<const char*>(lut_storage) + kLutBaseOffset;
    char* const stg_bytes = stage[wave];
    const PsStage<R>& stg = *reinterpret_cast<const PsStage<R>*>(stage[wave]);

    for (int u = wave; u < T; u += W) {  // uniform within the wave
        lds_wait_all();  // the previous round's reads of the stage and x buffer have landed
        ps_issue(stg_bytes, st.packed, st.ld_code, R, 0, u);
        WideScales<R> sc;
        ps_load_scales<R>(sc, st, 0, u, K, g);
        stage_x(xs[wave], st.x, u, M, K, 0, lane, 1);
        vm_wait_all();
        WideCodes<R> w;
        ps_readback<R>(stg, st, w);
        ps_round<DT, R, MM>(w, sc, lut, slot, xa, acc);
    }

#pragma unroll
    for (int q = 0; q < MM; ++q) red[wave][q][lane] = acc[0][q];
    __syncthreads();
    if (wave != 0) return;
#pragma unroll
    for (int w2 = 1; w2 < W; ++w2)
#pragma unroll
        for (int q = 0; q < MM; ++q) acc[0][q] += red[w2][q][lane];
    uint32_t bv[R];
    ps_load_bias<DT, R>(job, tile0, lane, bv);
    ps_store<DT, R, MM>(job, ybase, M, tile0, lane, acc, bv);
}

// ------------------------------------------------------------------------- 2-bit GEMV
//
// Decode GEMV (M <= 4) over 2-bit E8 weights (E8LatticePacker: four 2-bit codes per byte,
// one fp16 scale per gs weights): y = x . ((code - 1.5) * s)^T, fp32 accumulation, the
// group scale (in the activation dtype, as the native binding casts it,
// ojasx_math_bindings.cpp:286) applied to fp32 partial sums per group, as the reference's
// own 2-bit fused kernel does (ojasx_math_core.hpp:454-479: acc += group_acc * scale).
//
// Each wave owns one 16-row tile and walks K in 1024-k rounds.  A round of a row is 256
// code bytes (16 pieces of 16 bytes, 64 weights each) and 2048/gs scale bytes.  Lane (g, n)
// takes pieces g, 4 + g, 8 + g and 12 + g of row n: load t of the wave reads piece 4t + g of
// all 16 rows, so the four lane groups read 64 contiguous bytes of each row per
// instruction; scales use the same mapping (128/gs bytes per piece).  The next round's
// pieces are loaded into a second register set while the current round computes.
//
// Step J (0..31) of a round takes the 8 codes of half-word J % 8 of piece J / 8, k = 64 (4t +
// g) + 8 (J % 8).  Every 4-bit nibble (two codes) indexes a 16-entry table of weight pairs
// (code - 1.5 in the activation dtype, exact) with 32 copies: one conflict-free b32 read per
// pair of weights.  A row 4g' + m carries activation row m only in lane group g''s k slots
// (a zero block elsewhere), so the MFMA output of lane (g', n) is the partial sum of its own
// k slots and its group scale can multiply it every gs/8 steps; the four lane groups are
// added at the end.
//
// The byte table (BC copies, BC = 0: the nibble table): each code byte (four codes) indexes a
// 256-entry table of four weights (8 bytes) with BC copies, lane l reading copy l % BC: two
// b64 reads and two address computations per 8 weights instead of four of each.  16 copies
// (32 KB) leave two 4-wave workgroups per CU at M = 4; 32 copies (64 KB) make the reads
// conflict-free.

constexpr int kB2Waves = 4;
constexpr int kB2LutU4 = 16 * 32 * 4 / 16;  // 16 entries x 32 copies x 4 bytes
template <int BC>
constexpr int kB2ByteLutU4 = 256 * BC * 8 / 16;  // 256 entries x BC copies x 8 bytes
constexpr int kB2ZeroBytes = 2048;          // covers the largest A-fragment offset of a round

template <int DT>
__device__ __forceinline__ uint32_t b2_half(int c) {  // code c -> (c - 1.5) in dtype bits
    if constexpr (DT == kBF16) return c == 0 ? 0xBFC0u : c == 1 ? 0xBF00u : c == 2 ? 0x3F00u : 0x3FC0u;
    else return c == 0 ? 0xBE00u : c == 1 ? 0xB800u : c == 2 ? 0x3800u : 0x3E00u;
}

template <int DT, int NT>
__device__ __forceinline__ void fill_b2lut(uint4* lut) {
    for (int i = (int)threadIdx.x; i < kB2LutU4; i += NT) {
        const int e = i >> 3;  // 8 items (32 copies x 4 bytes) per entry
        const uint32_t w = b2_half<DT>(e & 3) | (b2_half<DT>(e >> 2) << 16);
        lut[i] = make_uint4(w, w, w, w);
    }
}

template <int DT, int NT, int BC>
__device__ __forceinline__ void fill_b2blut(uint4* lut) {
    for (int i = (int)threadIdx.x; i < kB2ByteLutU4<BC>; i += NT) {
        const int e = i / (BC / 2);  // BC / 2 items (BC copies x 8 bytes) per entry
        const uint32_t lo = b2_half<DT>(e & 3) | (b2_half<DT>((e >> 2) & 3) << 16);
        const uint32_t hi = b2_half<DT>((e >> 4) & 3) | (b2_half<DT>(e >> 6) << 16);
        lut[i] = make_uint4(lo, hi, lo, hi);
    }
}

// The table slot of a lane: 32 copies of 4 bytes, or 16 copies of 8 bytes (byte table).
template <int BC>
__device__ __forceinline__ uint32_t b2_slot(int lane) {
    return BC ? (uint32_t)(lane & (BC - 1)) * 8u : (uint32_t)(lane & 31) * 4u;
}

// B operand of the 8 codes in half-word H of dword dw: four nibble-table reads, or two
// byte-table reads.
template <int H, int BC>
__device__ __forceinline__ uint4 b2_operand(uint32_t dw, const char* lut, uint32_t slot) {
    if constexpr (BC != 0) {
        constexpr int sh = BC == 32 ? 8 : 7;  // entry stride BC x 8 bytes
        const uint32_t a0 = (__builtin_amdgcn_ubfe(dw, 16 * H, 8) << sh) | slot;
        const uint32_t a1 = (__builtin_amdgcn_ubfe(dw, 16 * H + 8, 8) << sh) | slot;
        const uint2 v0 = *reinterpret_cast<const uint2*>(lut + a0);
        const uint2 v1 = *reinterpret_cast<const uint2*>(lut + a1);
        return make_uint4(v0.x, v0.y, v1.x, v1.y);
    } else {
        uint32_t v[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint32_t a = (__builtin_amdgcn_ubfe(dw, 16 * H + 4 * i, 4) << 7) | slot;
            v[i] = *reinterpret_cast<const uint32_t*>(lut + a);
        }
        return make_uint4(v[0], v[1], v[2], v[3]);
    }
}

// Scale (fp16 bits) of step J for group size GS from this lane's scale pieces of the round.
template <int GS, int J>
__device__ __forceinline__ uint32_t b2_scale(const uint4 (&sp)[4]) {
    constexpr int t = J / 8, j = J % 8;           // piece, 8-weight unit within it
    constexpr int idx = (j * 8) / GS;             // scale within the piece
    constexpr int word = idx / 2, half = idx % 2;
    const uint32_t w = word == 0 ? sp[t].x : word == 1 ? sp[t].y : word == 2 ? sp[t].z : sp[t].w;
    return half ? (w >> 16) : (w & 0xFFFFu);
}

// The post-scaled B operand of step (piece T, 8-weight unit HW) from a lane's four code
// pieces: 2-bit, half-word HW of piece T through the nibble or byte table; 1-bit Root E8, code
// byte HW of piece T (8 bytes) through the 256-entry table of the code's 8 coordinates in the
// activation dtype (BC copies of 16 bytes, this lane's at `slot`).
template <int FMT, int T, int HW, int BC>
__device__ __forceinline__ uint4 post_operand(const uint4 (&cp)[4], const char* lut,
                                              uint32_t slot) {
    if constexpr (FMT == kFmtRoot) {
        const uint32_t code = ((HW < 4 ? cp[T].x : cp[T].y) >> (8 * (HW % 4))) & 0xFFu;
        return *reinterpret_cast<const uint4*>(lut + 16u * BC * code + slot);
    } else {
        const uint32_t dw = (HW / 2) == 0 ? cp[T].x : (HW / 2) == 1 ? cp[T].y
                          : (HW / 2) == 2 ? cp[T].z : cp[T].w;
        return b2_operand<(HW % 2), BC>(dw, lut, slot);
    }
}

// One round of R row tiles of one wave: steps 0..31, the A fragment read once per step for
// all R tiles, with the table reads and A fragment of step J + 1 issued before the MFMAs of
// step J and the scale of a finished group applied after the next group's first MFMA.
template <int DT, int MM, int GS, int R, int BC, int FMT = kFmt2Bit>
struct B2Round {
    static constexpr int kSpg = GS / 8;  // steps per scale group
    using Pieces = uint4[R][4];
    template <int J>
    __device__ __forceinline__ static void step(const Pieces& cp, const Pieces& sp,
                                                const char* lut, uint32_t slot,
                                                const char* xa, uint4& a_cur, uint4 (&b_cur)[R],
                                                f32x4 (&d)[R][2], float (&sf_prev)[R],
                                                float (&acc)[R][MM]) {
        uint4 a_n, b_n[R];
        if constexpr (J + 1 < 32) {
            constexpr int t = (J + 1) / 8, hw = (J + 1) % 8;
            a_n = *reinterpret_cast<const uint4*>(xa + 512 * t + 16 * hw);
#pragma unroll
            for (int r = 0; r < R; ++r) b_n[r] = post_operand<FMT, t, hw, BC>(cp[r], lut, slot);
        }
        constexpr int grp = J / kSpg, slot_d = grp & 1;
        constexpr bool first = (J % kSpg) == 0;
#pragma unroll
        for (int r = 0; r < R; ++r)
            d[r][slot_d] = mfma16<DT>(a_cur, b_cur[r],
                                      first ? f32x4{0.f, 0.f, 0.f, 0.f} : d[r][slot_d]);
#pragma unroll
        for (int r = 0; r < R; ++r) {
            if constexpr (first && J > 0) {
                // group grp - 1 is complete in the other accumulator
#pragma unroll
                for (int q = 0; q < MM; ++q)
                    acc[r][q] = __builtin_fmaf(d[r][slot_d ^ 1][q], sf_prev[r], acc[r][q]);
                keep_mfma_result(d[r][slot_d ^ 1], acc[r][0]);
            }
            if constexpr (first) sf_prev[r] = scale_for<DT>(b2_scale<GS, J>(sp[r]));
            if constexpr (J == 31) {
#pragma unroll
                for (int q = 0; q < MM; ++q)
                    acc[r][q] = __builtin_fmaf(d[r][slot_d][q], sf_prev[r], acc[r][q]);
                keep_mfma_result(d[r][slot_d], acc[r][0]);
            }
        }
        if constexpr (J + 1 < 32) {
            a_cur = a_n;
#pragma unroll
            for (int r = 0; r < R; ++r) b_cur[r] = b_n[r];
        }
    }
    template <int... J>
    __device__ __forceinline__ static void steps(const Pieces& cp, const Pieces& sp,
                                                 const char* lut, uint32_t slot, const char* xa,
                                                 uint4& a, uint4 (&b)[R], f32x4 (&d)[R][2],
                                                 float (&sf)[R], float (&acc)[R][MM],
                                                 std::integer_sequence<int, J...>) {
        (step<J>(cp, sp, lut, slot, xa, a, b, d, sf, acc), ...);
    }
    __device__ __forceinline__ static void run(const Pieces& cp, const Pieces& sp,
                                               const char* lut, uint32_t slot, const char* xa,
                                               float (&acc)[R][MM]) {
        uint4 a = *reinterpret_cast<const uint4*>(xa);
        uint4 b[R];
#pragma unroll
        for (int r = 0; r < R; ++r) b[r] = post_operand<FMT, 0, 0, BC>(cp[r], lut, slot);
        f32x4 d[R][2];
        float sf[R];
        steps(cp, sp, lut, slot, xa, a, b, d, sf, acc, std::make_integer_sequence<int, 32>{});
    }
};

// Stages round u of the MM activation rows into one wave's buffer: always 2 * MM DMA
// loads (rows m >= M re-read row M - 1 into slots no lane reads), so that every round
// issues the same number of loads.
template <int MM>
__device__ __forceinline__ void b2_stage_x(char* xs, __amdgpu_buffer_rsrc_t x, int64_t u, int M,
                                           int64_t K, int lane) {
#pragma unroll
    for (int q = 0; q < 2 * MM; ++q) {
        const int m = q >> 1, half = q & 1;
        const int msrc = m < M ? m : M - 1;
        __builtin_amdgcn_raw_ptr_buffer_load_lds(
            x, lds_ptr(xs + m * kXRow + half * 1024), 16,
            (uint32_t)(msrc * K * 2 + half * 1024 + lane * 16), uniform_offset(u * kRound * 2),
            0, 0);
    }
}

// Waits until the older of the two rounds in flight has landed.  A round issues 4 code
// loads, 4 scale loads (8 for GS 16) and 2 * MM activation loads; loads complete in issue
// order for vmcnt, so at most that many outstanding means every load of the older round
// is done.  s_waitcnt fields: vmcnt[3:0] and [15:14], expcnt[6:4] = 7 and lgkmcnt[11:8]
// = 15 (no wait).
template <int GS, int MM>
__device__ __forceinline__ void vm_wait_le_round() {
    constexpr int n = 4 + (GS == 16 ? 8 : 4) + 2 * MM;
    static_assert(n < 64, "vmcnt holds 6 bits");
    __builtin_amdgcn_s_waitcnt(0x0F70 | (n & 15) | ((n >> 4) << 14));
}

// This lane's scale pieces of round u (the 128 / gs scale bytes of code piece 4t + g).
template <int GS>
__device__ __forceinline__ void b2_scales(uint4 (&sp)[4], __amdgpu_buffer_rsrc_t sr,
                                          uint32_t vo_scale, int u) {
    const int so_s = uniform_offset((int64_t)u * 2048 / GS);
#pragma unroll
    for (int t = 0; t < 4; ++t) {
        constexpr uint32_t kPiece = 128 / GS;  // scale bytes per code piece
        const uint32_t o = vo_scale + 4u * kPiece * t;
        if constexpr (kPiece == 16) {
            const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(sr, o, so_s, 0);
            sp[t] = make_uint4(v.x, v.y, v.z, v.w);
        } else if constexpr (kPiece == 8) {
            const uint32_t lo = __builtin_amdgcn_raw_buffer_load_b32(sr, o, so_s, 0);
            const uint32_t hi = __builtin_amdgcn_raw_buffer_load_b32(sr, o + 4, so_s, 0);
            sp[t] = make_uint4(lo, hi, 0u, 0u);
        } else if constexpr (kPiece == 4) {
            sp[t] = make_uint4(__builtin_amdgcn_raw_buffer_load_b32(sr, o, so_s, 0), 0u, 0u, 0u);
        } else {
            sp[t] = make_uint4(__builtin_amdgcn_raw_buffer_load_b16(sr, o, so_s, 0), 0u, 0u, 0u);
        }
    }
}

// This lane's code and scale pieces of round u (t = 0..3: piece 4t + g).
template <int GS>
__device__ __forceinline__ void b2_load(uint4 (&cp)[4], uint4 (&sp)[4],
                                        __amdgpu_buffer_rsrc_t pr, __amdgpu_buffer_rsrc_t sr,
                                        uint32_t vo_code, uint32_t vo_scale, int u) {
    const int so_c = uniform_offset((int64_t)u * 256);
#pragma unroll
    for (int t = 0; t < 4; ++t) {
        const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(pr, vo_code + 64u * t, so_c, 0);
        cp[t] = make_uint4(v.x, v.y, v.z, v.w);
    }
    b2_scales<GS>(sp, sr, vo_scale, u);
}

// The same for 1-bit codes: four 8-byte pieces (one code byte per 8 weights) at the same k,
// piece 4t + g at byte 8 (4t + g) of the row's round (128 bytes); the scales as b2_load.
template <int GS>
__device__ __forceinline__ void b1_load(uint4 (&cp)[4], uint4 (&sp)[4],
                                        __amdgpu_buffer_rsrc_t pr, __amdgpu_buffer_rsrc_t sr,
                                        uint32_t vo_code, uint32_t vo_scale, int u) {
    const int so_c = uniform_offset((int64_t)u * 128);
#pragma unroll
    for (int t = 0; t < 4; ++t) {
        const auto v = __builtin_amdgcn_raw_buffer_load_b64(pr, vo_code + 32u * t, so_c, 0);
        cp[t] = make_uint4(v[0], v[1], 0u, 0u);
    }
    b2_scales<GS>(sp, sr, vo_scale, u);
}

// The 1-bit post-scaled table: code -> its 8 coordinates (0, +-1, +-2) in the activation
// dtype (16 bytes per code), built at compile time for bf16 and fp16 and copied into LDS.
constexpr uint32_t v1_half(bool bf16, int c) {
    return bf16 ? (c == 0 ? 0u : c == 1 ? 0x3F80u : c == 2 ? 0x4000u : c == -1 ? 0xBF80u : 0xC000u)
                : (c == 0 ? 0u : c == 1 ? 0x3C00u : c == 2 ? 0x4000u : c == -1 ? 0xBC00u : 0xC000u);
}

struct alignas(16) V1Tab {
    uint32_t w[kSel1Entries * 4];
};

constexpr V1Tab make_v1_tab(bool bf16) {
    V1Tab t{};
    const RootTable r = make_root_table();
    for (int e = 0; e < kSel1Entries; ++e)
        for (int h = 0; h < 4; ++h)
            t.w[4 * e + h] = v1_half(bf16, r.c[e][2 * h]) | (v1_half(bf16, r.c[e][2 * h + 1]) << 16);
    return t;
}

static __device__ const V1Tab kV1Tab[2] = {make_v1_tab(true), make_v1_tab(false)};

// Fills C copies of each entry (copy c of entry e at 16 (C e + c) bytes; lane l reads copy
// l % C, spreading a read's lanes over C bank groups) from the device table (an L2 hit
// after the first workgroup): every load of a thread is issued before its first write.
// NT: threads of the workgroup.
template <int DT, int C, int NT>
__device__ __forceinline__ void fill_v1(uint4* tab) {
    constexpr int kItems = kSel1Entries * C;
    constexpr int kPer = (kItems + NT - 1) / NT;
    const uint4* src = reinterpret_cast<const uint4*>(kV1Tab[DT == kBF16 ? 0 : 1].w);
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

// FMT: 2-bit codes (nibble table of values) or 1-bit Root E8 codes (one 4-KB table of each
// code's 8 coordinates, 8 code bytes per lane and round).
template <int DT, int MM, int GS, int FMT = kFmt2Bit>
__global__ __launch_bounds__(64 * kB2Waves) void gemv2_kernel(
    GemvLaunch args) {
    // this workgroup's linear: the launch's one job (per-linear launch) or a grouped job
    int64_t wg = blockIdx.x;
    const GemvJob job = gemv_job_of(args, wg);
    const void* const x = job.x ? job.x : args.x;
    const uint8_t* const packed = job.packed;
    const uint16_t* const scales = job.scales;
    const void* const bias = job.bias;
    void* const y = job.y ? job.y : args.y;
    const int M = args.M;
    const int64_t N = job.N, K = job.K;
    const LoraEp lora{job.lora_u, job.lora_b, job.lora_r,
                      job.lora_ldu ? job.lora_ldu : job.lora_r, job.N};
    static_assert(MM == 1 || MM == 4, "post-scaled layout holds at most 4 activation rows");
    static_assert(FMT == kFmt2Bit || FMT == kFmtRoot, "2-bit or 1-bit codes");
    constexpr bool kRoot = FMT == kFmtRoot;
    // 2-bit: the nibble table (filling the byte table's 32 KB costs a per-linear launch more
    // than its reads save: M = 1 per-linear 2-bit stack 0.497 -> 0.588 ms, same box)
    constexpr int BC = kRoot ? 1 : 0;
    __shared__ uint4 lut_storage[kRoot ? kSel1Entries : kB2LutU4];
    // Two activation buffers per wave, each its own LDS object ending in a zero block, so
    // that the compiler can tell the reads of one from the DMA into the other (it waits for
    // every outstanding load before an LDS read that may alias a pending DMA target).
    constexpr int kXsBytes = kB2Waves * MM * (int)kXRow;
    __shared__ __attribute__((aligned(16))) char xs0[kXsBytes + kB2ZeroBytes];
    __shared__ __attribute__((aligned(16))) char xs1[kXsBytes + kB2ZeroBytes];
    __shared__ float red[kB2Waves][MM][64];

    if constexpr (kRoot) fill_v1<DT, 1, 64 * kB2Waves>(lut_storage);
    else fill_b2lut<DT, 64 * kB2Waves>(lut_storage);
    for (int i = (int)threadIdx.x; i < kB2ZeroBytes / 16; i += 64 * kB2Waves) {
        reinterpret_cast<uint4*>(xs0 + kXsBytes)[i] = make_uint4(0u, 0u, 0u, 0u);
        reinterpret_cast<uint4*>(xs1 + kXsBytes)[i] = make_uint4(0u, 0u, 0u, 0u);
    }

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int g = lane >> 4, i16 = lane & 15;
    const int64_t tile = wg;
    const uint32_t rowbytes = (uint32_t)(kRoot ? K / 8 : K / 4);
    const uint32_t srowbytes = (uint32_t)(K * 2 / GS);
    const __amdgpu_buffer_rsrc_t pr = __builtin_amdgcn_make_buffer_rsrc(
        (void*)packed, (short)0, (int)(N * rowbytes), kRsrcWord3);
    const __amdgpu_buffer_rsrc_t sr = __builtin_amdgcn_make_buffer_rsrc(
        (void*)scales, (short)0, (int)(N * srowbytes), kRsrcWord3);
    const __amdgpu_buffer_rsrc_t xr = __builtin_amdgcn_make_buffer_rsrc(
        (void*)x, (short)0, (int)(M * K * 2), kRsrcWord3);
    const uint32_t row = (uint32_t)(tile * 16 + i16);
    const uint32_t vo_code = row * rowbytes + (kRoot ? 8u : 16u) * g;
    const uint32_t vo_scale = row * srowbytes + (128u / GS) * g;
    const uint32_t slot = kRoot ? 0u : b2_slot<BC>(lane);
    // this lane's codes and scales of round v (the same number of loads in both formats)
    auto load = [&](uint4 (&cp)[4], uint4 (&sp)[4], int v) {
        if constexpr (kRoot) b1_load<GS>(cp, sp, pr, sr, vo_code, vo_scale, v);
        else b2_load<GS>(cp, sp, pr, sr, vo_code, vo_scale, v);
    };

    // A row i16 = 4 g' + m: live in lane group g' only, for activation rows m < M
    const int am = i16 & 3;
    const bool a_live = (i16 >> 2) == g && am < M;
    const int xoff = wave * MM * (int)kXRow;
    char* const xw0 = xs0 + xoff;
    char* const xw1 = xs1 + xoff;
    const int aoff = a_live ? xoff + am * (int)kXRow + 128 * g : kXsBytes;
    const char* xa0 = xs0 + aoff;
    const char* xa1 = xs1 + aoff;

    // wave w takes rounds w, w + W, ...: its own register sets and activation buffers, so
    // the waves never wait for each other inside the loop
    const int T = (int)(K / kRound);
    float acc[1][MM];
#pragma unroll
    for (int q = 0; q < MM; ++q) acc[0][q] = 0.f;
    uint4 cp[2][1][4], sp[2][1][4];
    using Round = B2Round<DT, MM, GS, 1, BC, FMT>;
    int u = wave;
    if (u < T) {
        load(cp[0][0], sp[0][0], u);
        b2_stage_x<MM>(xw0, xr, u, M, K, lane);
    }
    __syncthreads();  // table and zero block ready
    const char* lut = reinterpret_cast<const char*>(lut_storage);
    // Rounds in pairs (u, u + W), each prefetching the next: the loop body has no branch
    // between the two halves, so the compiler neither sinks the prefetch of the second
    // half's codes below the first half's compute nor loses track of which activation
    // buffer a pending DMA writes (either would make it wait for the prefetch).  The last
    // pair or round runs after the loop, with nothing fetched behind it (a spare fetch
    // would add a memory round trip to the wave's end).
    while (u + 2 * kB2Waves < T) {  // uniform within the wave
        load(cp[1][0], sp[1][0], u + kB2Waves);
        b2_stage_x<MM>(xw1, xr, u + kB2Waves, M, K, lane);
        vm_wait_le_round<GS, MM>();  // round u's codes, scales and activations have landed
        Round::run(cp[0], sp[0], lut, slot, xa0, acc);
        lds_wait_all();  // this wave's reads of buffer 0 are done: it may be refilled
        load(cp[0][0], sp[0][0], u + 2 * kB2Waves);
        b2_stage_x<MM>(xw0, xr, u + 2 * kB2Waves, M, K, lane);
        vm_wait_le_round<GS, MM>();
        Round::run(cp[1], sp[1], lut, slot, xa1, acc);
        lds_wait_all();
        u += 2 * kB2Waves;
    }
    if (u + kB2Waves < T) {  // a last pair
        load(cp[1][0], sp[1][0], u + kB2Waves);
        b2_stage_x<MM>(xw1, xr, u + kB2Waves, M, K, lane);
        vm_wait_le_round<GS, MM>();
        Round::run(cp[0], sp[0], lut, slot, xa0, acc);
        vm_wait_all();
        Round::run(cp[1], sp[1], lut, slot, xa1, acc);
    } else if (u < T) {  // a last round
        vm_wait_all();
        Round::run(cp[0], sp[0], lut, slot, xa0, acc);
    }

    // add the waves' partial sums, then the four lane groups; lane group q stores row q
#pragma unroll
    for (int q = 0; q < MM; ++q) red[wave][q][lane] = acc[0][q];
    __syncthreads();
    if (wave != 0) return;
    float out = 0.f;
#pragma unroll
    for (int q = 0; q < MM; ++q) {
        float v = red[0][q][lane];
#pragma unroll
        for (int w2 = 1; w2 < kB2Waves; ++w2) v += red[w2][q][lane];
        v += __shfl_xor(v, 16);
        v += __shfl_xor(v, 32);
        if (q == g) out = v;
    }
    if ((int64_t)row < N && g < M) {
        const float bv = bias ? load_as_f32<DT>(bias, row) : 0.f;
        store_from_f32<DT>(y, (int64_t)g * job.y_ld + job.y_col + row,
                           out + bv + lora_term<DT>(lora, g, row));
    }
}

// ------------------------------------------------------------------------- 2-bit GEMV, 4 < M <= 16
//
// With up to 16 activation rows every A row of the MFMA is live, so the group scale can no
// longer multiply per-lane partial sums: the B operand carries the weights themselves,
// rnd_dt((c - 1.5) * s_dt) (lattice.py:274-276; the native binding's dtype rule,
// ojasx_math_bindings.cpp:286).  Per scale group a lane forms the two value words of
// `values2`; each pair of codes (one nibble) then becomes one dword of two weights by
// v_perm_b32, its selector read from a 16-entry nibble table (32 copies: one conflict-free
// b32 read per pair of weights).
//
// Each workgroup owns one 16-row tile; its 4 waves take the 256-k rounds u = w, w + 4, ...
// (their own registers and activation buffers, so they never wait for each other until the
// final reduction).  A round of a row is 64 code bytes and 512/gs scale bytes: lane (g, n)
// takes code bytes 16g .. 16g+15 of row n (one 16-byte load per lane; the four lane groups
// read 64 contiguous bytes of each row per instruction) and the 64/gs scales of those
// weights.  The 16 activation rows of the round (8 KB) are staged into the wave's LDS
// buffer by eight 1-KB loads.  Step h (0..7) takes the 8 codes of half-word h of the lane's
// piece, k = 256u + 64g + 8h, and runs one v_mfma_f32_16x16x32 with activation row i16 as
// A row i16 (rows past M re-read row M - 1; their outputs are not stored).

constexpr int kB2mRound = 256;                      // K per round
constexpr int kB2mXBytes = 16 * kB2mRound * 2;      // one wave's activation buffer (8 KB)

template <int NT>
__device__ __forceinline__ void fill_b2sel(uint4* lut) {
    for (int i = (int)threadIdx.x; i < kB2LutU4; i += NT) {
        const uint32_t e = (uint32_t)i >> 3;  // nibble: code c0 in bits 0-1, c1 in bits 2-3
        const uint32_t c0 = e & 3u, c1 = e >> 2;
        const uint32_t w = (2u * c0) | ((2u * c0 + 1u) << 8) | ((2u * c1) << 16) |
                           ((2u * c1 + 1u) << 24);
        lut[i] = make_uint4(w, w, w, w);
    }
}

// The byte form (BC copies, as the post-scaled byte table): a code byte -> the selector
// words of its two nibbles (8 bytes), one b64 read per four weights.
template <int NT, int BC>
__device__ __forceinline__ void fill_b2bsel(uint4* lut) {
    auto sel = [](uint32_t n) {
        const uint32_t c0 = n & 3u, c1 = n >> 2;
        return (2u * c0) | ((2u * c0 + 1u) << 8) | ((2u * c1) << 16) | ((2u * c1 + 1u) << 24);
    };
    for (int i = (int)threadIdx.x; i < kB2ByteLutU4<BC>; i += NT) {
        const uint32_t e = (uint32_t)i / (BC / 2);
        const uint32_t lo = sel(e & 15u), hi = sel(e >> 4);
        lut[i] = make_uint4(lo, hi, lo, hi);
    }
}

// B operand (8 weights) of half-word H of this lane's 16-byte code piece: nibble selectors
// (BC = 0) or byte selector pairs.
template <int H, int BC = 0>
__device__ __forceinline__ uint4 b2m_operand(const uint4& cp, const uint2& val, const char* lut,
                                             uint32_t slot) {
    const uint32_t dw = (H / 2) == 0 ? cp.x : (H / 2) == 1 ? cp.y : (H / 2) == 2 ? cp.z : cp.w;
    uint32_t v[4];
    if constexpr (BC != 0) {
        constexpr int sh = BC == 32 ? 8 : 7;
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const uint32_t a = (__builtin_amdgcn_ubfe(dw, 16 * (H % 2) + 8 * j, 8) << sh) | slot;
            const uint2 sel = *reinterpret_cast<const uint2*>(lut + a);
            v[2 * j] = __builtin_amdgcn_perm(val.x, val.y, sel.x);
            v[2 * j + 1] = __builtin_amdgcn_perm(val.x, val.y, sel.y);
        }
    } else {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint32_t a = (__builtin_amdgcn_ubfe(dw, 16 * (H % 2) + 4 * i, 4) << 7) | slot;
            const uint32_t sel = *reinterpret_cast<const uint32_t*>(lut + a);
            v[i] = __builtin_amdgcn_perm(val.x, val.y, sel);
        }
    }
    return make_uint4(v[0], v[1], v[2], v[3]);
}

// B operand (8 weights) of 1-bit code byte H of this lane's 8 code bytes: the code's four
// selector words from the 256-entry table (C copies, this lane's at byte `slot` of an
// entry), applied to the group's value words.
template <int H, int C = 1>
__device__ __forceinline__ uint4 root_operand(const uint4& cp, const uint2& val, const char* tab,
                                              uint32_t slot = 0) {
    const uint32_t byte = ((H < 4 ? cp.x : cp.y) >> (8 * (H % 4))) & 0xFFu;
    const uint4 sel = *reinterpret_cast<const uint4*>(tab + 16u * C * byte + slot);
    return make_uint4(__builtin_amdgcn_perm(val.x, val.y, sel.x),
                      __builtin_amdgcn_perm(val.x, val.y, sel.y),
                      __builtin_amdgcn_perm(val.x, val.y, sel.z),
                      __builtin_amdgcn_perm(val.x, val.y, sel.w));
}

// B operand (8 weights) of ternary code H of this lane's 8 codes (12 bytes in cp.x..z): the
// two half-code mask entries of the bank-sliced table (e8t_lut.h) AND-ed with the group's
// scale word s | s << 16 | 0x80008000 (val.x).
template <int H>
__device__ __forceinline__ uint4 ternary_operand(const uint4& cp, const uint2& val,
                                                 const char* lut, uint32_t slot) {
    const uint32_t d[3] = {cp.x, cp.y, cp.z};
    const uint32_t z = code_z<H>(d, slot);
    const uint32_t h = __umulhi(z, kHiMagic);
    const uint2 ml = *reinterpret_cast<const uint2*>(lut + lo_addr_of(h, z));
    const uint2 mh = *reinterpret_cast<const uint2*>(lut + (h * kLutStride + slot));
    const uint32_t s = val.x;
    return make_uint4(ml.x & s, ml.y & s, mh.x & s, mh.y & s);
}

// Value words of a scale group in format FMT: 2-bit or 1-bit Root E8 as above; ternary the
// mask AND word of the one scale.
template <int DT, int FMT>
__device__ __forceinline__ uint2 values_of(uint32_t s16) {
    if constexpr (FMT == kFmtRoot) return values1<DT>(s16);
    else if constexpr (FMT == kFmt2Bit) return values2<DT>(s16);
    else {
        uint32_t w0, w1;
        scale_words<DT>(s16, w0, w1);
        return make_uint2(w0, 0u);
    }
}

template <int FMT, int H, int BC = 0>
__device__ __forceinline__ uint4 operand_of(const uint4& cp, const uint2& val, const char* lut,
                                            uint32_t slot) {
    if constexpr (FMT == kFmtRoot)  // the single-copy table has no slot
        return root_operand<H, (BC ? BC : 1)>(cp, val, lut, BC ? slot : 0u);
    else if constexpr (FMT == kFmt2Bit) return b2m_operand<H, BC>(cp, val, lut, slot);
    else return ternary_operand<H>(cp, val, lut, slot);
}

// Scale (fp16 bits) of step H from this lane's scales of the round (64/GS of them).
template <int GS, int H>
__device__ __forceinline__ uint32_t b2m_scale(const uint4& sp) {
    constexpr int idx = (8 * H) / GS, word = idx / 2;
    const uint32_t w = word == 0 ? sp.x : word == 1 ? sp.y : word == 2 ? sp.z : sp.w;
    return (idx % 2) ? (w >> 16) : (w & 0xFFFFu);
}

// Step h's A fragment: with the lane's offset xo = 8192 w + 512 i16 + 16 ((8g & 16) |
// ((8g & 8) ^ (i16 & 8)) | (i16 & 7)) (bits 4..6 equal to i16 & 7), piece 8g + h of row
// i16 sits at xs + (xo ^ 16 h).
// Row tiles per workgroup: one below kB2mTwoTilesFrom row tiles (these launches need the
// workgroups), two from there (half the staged activation bytes per weight).  Measured on
// MI355X, per-linear M = 16 (same box): gate/up 17.0 -> 13.5 us with two; four 14.2 us;
// two from 256 tiles on (q/o, down) 5.7 -> 7.4 and 13.9 -> 18.8 us.
constexpr int64_t kB2mTwoTilesFrom = 512;

template <int DT, int GS, int FMT, int R, int BC = 0>
struct B2mRound {
    // step H: the A fragment and B operands of step H + 1 are formed before the MFMAs of
    // step H are issued; the R tiles share the A fragment
    template <int H>
    __device__ __forceinline__ static void step(const uint4 (&cp)[R], const uint4 (&sp)[R],
                                                const char* lut, uint32_t slot, const char* xs,
                                                uint32_t xo, uint4& a_cur, uint4 (&b_cur)[R],
                                                uint2 (&val)[R], f32x4 (&acc)[R]) {
        uint4 a_n, b_n[R];
        if constexpr (H + 1 < 8) {
#pragma unroll
            for (int r = 0; r < R; ++r) {
                if constexpr ((8 * (H + 1)) % GS == 0)
                    val[r] = values_of<DT, FMT>(b2m_scale<GS, H + 1>(sp[r]));
                b_n[r] = operand_of<FMT, H + 1, BC>(cp[r], val[r], lut, slot);
            }
            a_n = *reinterpret_cast<const uint4*>(xs + (xo ^ (16u * (H + 1))));
        }
#pragma unroll
        for (int r = 0; r < R; ++r) acc[r] = mfma16<DT>(a_cur, b_cur[r], acc[r]);
        if constexpr (H + 1 < 8) {
            a_cur = a_n;
#pragma unroll
            for (int r = 0; r < R; ++r) b_cur[r] = b_n[r];
        }
    }
    template <int... H>
    __device__ __forceinline__ static void steps(const uint4 (&cp)[R], const uint4 (&sp)[R],
                                                 const char* lut, uint32_t slot, const char* xs,
                                                 uint32_t xo, uint4& a, uint4 (&b)[R],
                                                 uint2 (&val)[R], f32x4 (&acc)[R],
                                                 std::integer_sequence<int, H...>) {
        (step<H>(cp, sp, lut, slot, xs, xo, a, b, val, acc), ...);
    }
    __device__ __forceinline__ static void run(const uint4 (&cp)[R], const uint4 (&sp)[R],
                                               const char* lut, uint32_t slot, const char* xs,
                                               uint32_t xo, f32x4 (&acc)[R]) {
        uint2 val[R];
        uint4 b[R];
#pragma unroll
        for (int r = 0; r < R; ++r) {
            val[r] = values_of<DT, FMT>(b2m_scale<GS, 0>(sp[r]));
            b[r] = operand_of<FMT, 0, BC>(cp[r], val[r], lut, slot);
        }
        uint4 a = *reinterpret_cast<const uint4*>(xs + xo);
        steps(cp, sp, lut, slot, xs, xo, a, b, val, acc, std::make_integer_sequence<int, 8>{});
    }
};

// Activation buffer layout: row m (512 bytes) at 512 m; its 16-byte piece p (k = 8p ..
// 8p + 7 of the round) at position (p & 16) | ((p & 15) ^ m), so that the 16 rows' reads of
// one piece fall on distinct banks.  The DMA writes 64 consecutive 16-byte slots per load
// (rows 2q and 2q + 1), so lane l of load q fetches the piece that belongs at its slot.
// Global byte offset (without the round) of lane l's piece in load q (rows >= M re-read row
// M - 1; no lane reads their outputs).
__device__ __forceinline__ uint32_t b2m_x_offset(int q, int lane, int M, int64_t K) {
    const uint32_t m = 2u * (uint32_t)q + ((uint32_t)lane >> 5), pos = (uint32_t)lane & 31u;
    const uint32_t p = (pos & 16u) | ((pos & 15u) ^ m);
    const uint32_t msrc = (int)m < M ? m : (uint32_t)(M - 1);
    return msrc * (uint32_t)(K * 2) + 16u * p;
}

// Stages round u of the 16 activation rows into one wave's buffer: eight 1-KB loads, the
// same count every round.
__device__ __forceinline__ void b2m_stage_x(char* xs, __amdgpu_buffer_rsrc_t x, int64_t u,
                                            const uint32_t (&xo)[8]) {
#pragma unroll
    for (int q = 0; q < 8; ++q)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(x, lds_ptr(xs + 1024 * q), 16, xo[q],
                                                 uniform_offset(u * kB2mRound * 2), 0, 0);
}

// Waits until the older of the two rounds in flight has landed: a round issues one code
// and one scale load per tile and eight activation loads (in-order vmcnt).
template <int R>
__device__ __forceinline__ void b2m_wait_round() {
    constexpr int n = 2 * R + 8;
    __builtin_amdgcn_s_waitcnt(0x0F70 | (n & 15) | ((n >> 4) << 14));
}

// This lane's code piece and scales of round u.
template <int GS, int FMT>
__device__ __forceinline__ void b2m_load(uint4& cp, uint4& sp, __amdgpu_buffer_rsrc_t pr,
                                         __amdgpu_buffer_rsrc_t sr, uint32_t vo_code,
                                         uint32_t vo_scale, int u) {
    if constexpr (FMT == kFmtRoot) {  // 8 code bytes (64 weights)
        const auto v = __builtin_amdgcn_raw_buffer_load_b64(pr, vo_code,
                                                            uniform_offset((int64_t)u * 32), 0);
        cp = make_uint4(v[0], v[1], 0u, 0u);
    } else if constexpr (FMT == kFmtTernary) {  // 12 code bytes (8 codes, 64 weights)
        const u32x3 v = __builtin_amdgcn_raw_buffer_load_b96(pr, vo_code,
                                                             uniform_offset((int64_t)u * 48), 0);
        cp = make_uint4(v.x, v.y, v.z, 0u);
    } else {                          // 16 code bytes (64 weights)
        const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(pr, vo_code,
                                                              uniform_offset((int64_t)u * 64), 0);
        cp = make_uint4(v.x, v.y, v.z, v.w);
    }
    const int so = uniform_offset((int64_t)u * (2 * kB2mRound / GS));
    if constexpr (GS == 8) {
        const u32x4 s = __builtin_amdgcn_raw_buffer_load_b128(sr, vo_scale, so, 0);
        sp = make_uint4(s.x, s.y, s.z, s.w);
    } else if constexpr (GS == 16) {
        const auto s = __builtin_amdgcn_raw_buffer_load_b64(sr, vo_scale, so, 0);
        sp = make_uint4(s[0], s[1], 0u, 0u);
    } else if constexpr (GS == 32) {
        sp = make_uint4(__builtin_amdgcn_raw_buffer_load_b32(sr, vo_scale, so, 0), 0u, 0u, 0u);
    } else {
        sp = make_uint4(__builtin_amdgcn_raw_buffer_load_b16(sr, vo_scale, so, 0), 0u, 0u, 0u);
    }
}

template <int DT, int GS, int FMT, int R>
__global__ __launch_bounds__(64 * kB2Waves) void gemv2m_kernel(
    GemvLaunch args) {
    // this workgroup's linear: the launch's one job (per-linear launch) or a grouped job
    int64_t wg = blockIdx.x;
    const GemvJob job = gemv_job_of(args, wg);
    const void* const x = job.x ? job.x : args.x;
    const uint8_t* const packed = job.packed;
    const uint16_t* const scales = job.scales;
    const void* const bias = job.bias;
    void* const y = job.y ? job.y : args.y;
    const int M = args.M;
    const int64_t N = job.N, K = job.K;
    const LoraEp lora{job.lora_u, job.lora_b, job.lora_r,
                      job.lora_ldu ? job.lora_ldu : job.lora_r, job.N};
    static_assert(GS == 8 || GS == 16 || GS == 32 || GS == 64, "group size 8..64");
    static_assert(FMT == kFmtTernary || FMT == kFmt2Bit || FMT == kFmtRoot, "code format");
    static_assert(FMT != kFmtTernary || GS >= 16, "ternary group sizes are multiples of 16");
    // ternary: half-code masks (bank-sliced); 2-bit: nibble -> selector (32 copies); 1-bit:
    // code -> four selectors
    __shared__ uint4 lut_storage[FMT == kFmtTernary ? kLutValidStorageU4
                                 : FMT == kFmtRoot  ? kSel1Entries
                                                    : kB2LutU4];
    // two activation buffers per wave, separate LDS objects (see gemv2_kernel)
    __shared__ __attribute__((aligned(128))) char xs0[kB2Waves * kB2mXBytes];
    __shared__ __attribute__((aligned(128))) char xs1[kB2Waves * kB2mXBytes];
    static_assert(R * 64 * 16 <= kB2mXBytes, "partial sums fit a wave's activation buffer");

    if constexpr (FMT == kFmtTernary)
        fill_lut<64 * kB2Waves, kLutValidEntries>(lut_storage, kLutMasks);
    else if constexpr (FMT == kFmtRoot) fill_sel1<64 * kB2Waves>(lut_storage);
    else fill_b2sel<64 * kB2Waves>(lut_storage);

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int g = lane >> 4, i16 = lane & 15;
    const int64_t tile = wg;
    // code bytes per row, and per lane group (64 weights) of a round
    const uint32_t rowbytes = (uint32_t)(FMT == kFmtTernary ? K * 3 / 16
                                         : FMT == kFmtRoot  ? K / 8 : K / 4);
    constexpr uint32_t kLaneBytes = FMT == kFmtTernary ? 12u : FMT == kFmtRoot ? 8u : 16u;
    const uint32_t srowbytes = (uint32_t)(K * 2 / GS);
    const __amdgpu_buffer_rsrc_t pr = __builtin_amdgcn_make_buffer_rsrc(
        (void*)packed, (short)0, (int)(N * rowbytes), kRsrcWord3);
    const __amdgpu_buffer_rsrc_t sr = __builtin_amdgcn_make_buffer_rsrc(
        (void*)scales, (short)0, (int)(N * srowbytes), kRsrcWord3);
    const __amdgpu_buffer_rsrc_t xr = __builtin_amdgcn_make_buffer_rsrc(
        (void*)x, (short)0, (int)(M * K * 2), kRsrcWord3);
    // rows past N read zeros (buffer bound) and are never stored
    uint32_t vo_code[R], vo_scale[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const uint32_t row_r = (uint32_t)((tile * R + r) * 16 + i16);
        vo_code[r] = row_r * rowbytes + kLaneBytes * g;
        vo_scale[r] = row_r * srowbytes + (128u / GS) * g;
    }
    const uint32_t slot = FMT == kFmtTernary ? (uint32_t)(lane & (kLutSlots - 1)) * 8u
                                             : (uint32_t)(lane & 31) * 4u;
    uint32_t xo_ld[8];
#pragma unroll
    for (int q = 0; q < 8; ++q) xo_ld[q] = b2m_x_offset(q, lane, M, K);
    const uint32_t gu = (uint32_t)g, iu = (uint32_t)i16;
    const uint32_t xo = (uint32_t)wave * kB2mXBytes + 512u * iu +
                        16u * ((8u * gu & 16u) | ((8u * gu & 8u) ^ (iu & 8u)) | (iu & 7u));
    char* const xw0 = xs0 + wave * kB2mXBytes;
    char* const xw1 = xs1 + wave * kB2mXBytes;

    // wave w takes rounds w, w + W, ...; round u + W is fetched while round u computes
    const int T = (int)(K / kB2mRound);
    f32x4 acc[R];
#pragma unroll
    for (int r = 0; r < R; ++r) acc[r] = f32x4{0.f, 0.f, 0.f, 0.f};
    uint4 cp[2][R], sp[2][R];
    int u = wave;
    if (u < T) {
        #pragma unroll
        for (int r = 0; r < R; ++r)
            b2m_load<GS, FMT>(cp[0][r], sp[0][r], pr, sr, vo_code[r], vo_scale[r], u);
        b2m_stage_x(xw0, xr, u, xo_ld);
    }
    __syncthreads();  // selector table ready
    const char* lut = reinterpret_cast<const char*>(lut_storage) +
                      (FMT == kFmtTernary ? kLutBaseOffset : 0u);
    // rounds in pairs, as in gemv2_kernel (the last pair or round after the loop)
    while (u + 2 * kB2Waves < T) {  // uniform within the wave
        #pragma unroll
        for (int r = 0; r < R; ++r)
            b2m_load<GS, FMT>(cp[1][r], sp[1][r], pr, sr, vo_code[r], vo_scale[r], u + kB2Waves);
        b2m_stage_x(xw1, xr, u + kB2Waves, xo_ld);
        b2m_wait_round<R>();  // round u's codes, scales and activations have landed
        B2mRound<DT, GS, FMT, R>::run(cp[0], sp[0], lut, slot, xs0, xo, acc);
        lds_wait_all();  // this wave's reads of buffer 0 are done: it may be refilled
        #pragma unroll
        for (int r = 0; r < R; ++r)
            b2m_load<GS, FMT>(cp[0][r], sp[0][r], pr, sr, vo_code[r], vo_scale[r],
                              u + 2 * kB2Waves);
        b2m_stage_x(xw0, xr, u + 2 * kB2Waves, xo_ld);
        b2m_wait_round<R>();
        B2mRound<DT, GS, FMT, R>::run(cp[1], sp[1], lut, slot, xs1, xo, acc);
        lds_wait_all();
        u += 2 * kB2Waves;
    }
    if (u + kB2Waves < T) {  // a last pair
        #pragma unroll
        for (int r = 0; r < R; ++r)
            b2m_load<GS, FMT>(cp[1][r], sp[1][r], pr, sr, vo_code[r], vo_scale[r], u + kB2Waves);
        b2m_stage_x(xw1, xr, u + kB2Waves, xo_ld);
        b2m_wait_round<R>();
        B2mRound<DT, GS, FMT, R>::run(cp[0], sp[0], lut, slot, xs0, xo, acc);
        vm_wait_all();
        B2mRound<DT, GS, FMT, R>::run(cp[1], sp[1], lut, slot, xs1, xo, acc);
    } else if (u < T) {  // a last round
        vm_wait_all();
        B2mRound<DT, GS, FMT, R>::run(cp[0], sp[0], lut, slot, xs0, xo, acc);
    }

    // add the waves' partial sums (each wave's in its own, no longer read, part of buffer 0);
    // lane (g, n) holds rows m = 4g + q of column n
    f32x4* const red = reinterpret_cast<f32x4*>(xs0);
    constexpr int kRedWave = kB2mXBytes / 16;  // f32x4 slots per wave
#pragma unroll
    for (int r = 0; r < R; ++r) red[wave * kRedWave + r * 64 + lane] = acc[r];
    __syncthreads();
    if (wave != 0) return;
#pragma unroll
    for (int r = 0; r < R; ++r) {
#pragma unroll
        for (int w2 = 1; w2 < kB2Waves; ++w2) {
            const f32x4 o = red[w2 * kRedWave + r * 64 + lane];
            acc[r][0] += o[0];
            acc[r][1] += o[1];
            acc[r][2] += o[2];
            acc[r][3] += o[3];
        }
        const int64_t row = (tile * R + r) * 16 + i16;
        if (row < N) {
            const float bv = bias ? load_as_f32<DT>(bias, row) : 0.f;
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const int m = 4 * g + q;
                if (m < M)
                    store_from_f32<DT>(y, (int64_t)m * job.y_ld + job.y_col + row,
                                       acc[r][q] + bv + lora_term<DT>(lora, m, row));
            }
        }
    }
}


// ---- the B-operand GEMV at M <= 4: four activation rows staged, four rounds in flight
//
// At M <= 4 the kernel above still stages 16 activation rows per round (8 KB of its wave's
// LDS), which is what limits it to two rounds in flight.  Staging only rows 0..3 (2 KB per
// round; A rows i16 >= 4 read row i16 & 3, and no lane stores their outputs) leaves room for
// four rounds per wave in four buffers, so a wave of a decode-sized layer (K = 4096: four
// rounds) requests all of its weights at once.  Spare slots past a wave's last round load
// from past every buffer's end: zeros, no memory traffic, and the same count of loads per
// slot, so that one wait count fits every slot.
constexpr int kB2sRows = 4;
constexpr int kB2sXBytes = kB2sRows * kB2mRound * 2;  // 2 KB per wave and round

// b2m_load of round u, or (live == false) the same loads past the buffers' ends.
template <int GS, int FMT>
__device__ __forceinline__ void b2s_load(uint4& cp, uint4& sp, __amdgpu_buffer_rsrc_t pr,
                                         __amdgpu_buffer_rsrc_t sr, uint32_t vo_code,
                                         uint32_t vo_scale, int u, bool live) {
    const uint32_t vc = live ? vo_code : kNoRecordOffset, vs = live ? vo_scale : kNoRecordOffset;
    constexpr int kCodeRound = FMT == kFmtRoot ? 32 : FMT == kFmtTernary ? 48 : 64;
    const int sc = live ? uniform_offset((int64_t)u * kCodeRound) : 0;
    const int ss = live ? uniform_offset((int64_t)u * (2 * kB2mRound / GS)) : 0;
    if constexpr (FMT == kFmtRoot) {
        const auto v = __builtin_amdgcn_raw_buffer_load_b64(pr, vc, sc, 0);
        cp = make_uint4(v[0], v[1], 0u, 0u);
    } else if constexpr (FMT == kFmtTernary) {
        const u32x3 v = __builtin_amdgcn_raw_buffer_load_b96(pr, vc, sc, 0);
        cp = make_uint4(v.x, v.y, v.z, 0u);
    } else {
        const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(pr, vc, sc, 0);
        cp = make_uint4(v.x, v.y, v.z, v.w);
    }
    if constexpr (GS == 8) {
        const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(sr, vs, ss, 0);
        sp = make_uint4(v.x, v.y, v.z, v.w);
    } else if constexpr (GS == 16) {
        const auto v = __builtin_amdgcn_raw_buffer_load_b64(sr, vs, ss, 0);
        sp = make_uint4(v[0], v[1], 0u, 0u);
    } else if constexpr (GS == 32) {
        sp = make_uint4(__builtin_amdgcn_raw_buffer_load_b32(sr, vs, ss, 0), 0u, 0u, 0u);
    } else {
        sp = make_uint4(__builtin_amdgcn_raw_buffer_load_b16(sr, vs, ss, 0), 0u, 0u, 0u);
    }
}

// Issues one round's loads into pipeline slot buffer `xb` (this wave's part of it).  (Not
// a template: the host pass rejects the LDS-load builtin in a kernel template's callee.)
__device__ __forceinline__ void b2s_stage_x(char* xb, __amdgpu_buffer_rsrc_t x, uint32_t xo0,
                                            uint32_t xo1, int so) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(x, lds_ptr(xb), 16, xo0, so, 0, 0);
    __builtin_amdgcn_raw_ptr_buffer_load_lds(x, lds_ptr(xb + 1024), 16, xo1, so, 0, 0);
}

template <int DT, int GS, int FMT, int R>
__global__ __launch_bounds__(64 * kB2Waves) void gemv2s_kernel(
    GemvLaunch args) {
    // this workgroup's linear: the launch's one job (per-linear launch) or a grouped job
    int64_t wg = blockIdx.x;
    const GemvJob job = gemv_job_of(args, wg);
    const void* const x = job.x ? job.x : args.x;
    const uint8_t* const packed = job.packed;
    const uint16_t* const scales = job.scales;
    const void* const bias = job.bias;
    void* const y = job.y ? job.y : args.y;
    const int M = args.M;
    const int64_t N = job.N, K = job.K;
    const LoraEp lora{job.lora_u, job.lora_b, job.lora_r,
                      job.lora_ldu ? job.lora_ldu : job.lora_r, job.N};
    static_assert(GS == 8 || GS == 16 || GS == 32 || GS == 64, "group size 8..64");
    static_assert(FMT == kFmtTernary || FMT == kFmt2Bit || FMT == kFmtRoot, "code format");
    static_assert(FMT != kFmtTernary || GS >= 16, "ternary group sizes are multiples of 16");
    static_assert(R * 64 * 16 <= kB2sXBytes, "partial sums fit a wave's activation buffer");
    constexpr int L = 2 * R + 2;  // loads per round: codes and scales per tile, 2 of rows
    __shared__ uint4 lut_storage[FMT == kFmtTernary ? kLutValidStorageU4
                                 : FMT == kFmtRoot  ? kSel1Entries
                                                    : kB2LutU4];
    // four pipeline buffers, separate LDS objects (the compiler then knows that a read of
    // one does not wait for loads into another)
    __shared__ __attribute__((aligned(128))) char xs0[kB2Waves * kB2sXBytes];
    __shared__ __attribute__((aligned(128))) char xs1[kB2Waves * kB2sXBytes];
    __shared__ __attribute__((aligned(128))) char xs2[kB2Waves * kB2sXBytes];
    __shared__ __attribute__((aligned(128))) char xs3[kB2Waves * kB2sXBytes];

    if constexpr (FMT == kFmtTernary)
        fill_lut<64 * kB2Waves, kLutValidEntries>(lut_storage, kLutMasks);
    else if constexpr (FMT == kFmtRoot) fill_sel1<64 * kB2Waves>(lut_storage);
    else fill_b2sel<64 * kB2Waves>(lut_storage);

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int g = lane >> 4, i16 = lane & 15;
    const int64_t tile = wg;
    const uint32_t rowbytes = (uint32_t)(FMT == kFmtTernary ? K * 3 / 16
                                         : FMT == kFmtRoot  ? K / 8 : K / 4);
    constexpr uint32_t kLaneBytes = FMT == kFmtTernary ? 12u : FMT == kFmtRoot ? 8u : 16u;
    const uint32_t srowbytes = (uint32_t)(K * 2 / GS);
    const __amdgpu_buffer_rsrc_t pr = __builtin_amdgcn_make_buffer_rsrc(
        (void*)packed, (short)0, (int)(N * rowbytes), kRsrcWord3);
    const __amdgpu_buffer_rsrc_t sr = __builtin_amdgcn_make_buffer_rsrc(
        (void*)scales, (short)0, (int)(N * srowbytes), kRsrcWord3);
    const __amdgpu_buffer_rsrc_t xr = __builtin_amdgcn_make_buffer_rsrc(
        (void*)x, (short)0, (int)(M * K * 2), kRsrcWord3);
    // rows past N read zeros (buffer bound) and are never stored
    uint32_t vo_code[R], vo_scale[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const uint32_t row_r = (uint32_t)((tile * R + r) * 16 + i16);
        vo_code[r] = row_r * rowbytes + kLaneBytes * g;
        vo_scale[r] = row_r * srowbytes + (128u / GS) * g;
    }
    const uint32_t slot = FMT == kFmtTernary ? (uint32_t)(lane & (kLutSlots - 1)) * 8u
                                             : (uint32_t)(lane & 31) * 4u;
    // activation rows 0..3 (rows >= M re-read row M - 1); the buffer layout of gemv2m_kernel
    const uint32_t xo_ld0 = b2m_x_offset(0, lane, M, K), xo_ld1 = b2m_x_offset(1, lane, M, K);
    // A row i16 reads row i16 & 3: piece 8g + h at position 8g + (m ^ h) of row m
    const uint32_t am = (uint32_t)i16 & 3u;
    const uint32_t xo = (uint32_t)wave * kB2sXBytes + 512u * am + 128u * (uint32_t)g + 16u * am;

    // wave w takes rounds u = w + W i, i = 0 .. nr - 1, four of them in flight
    const int T = (int)(K / kB2mRound);
    const int nr = wave < T ? (T - 1 - wave) / kB2Waves + 1 : 0;
    f32x4 acc[R];
#pragma unroll
    for (int r = 0; r < R; ++r) acc[r] = f32x4{0.f, 0.f, 0.f, 0.f};
    uint4 cp[4][R], sp[4][R];
    char* const xsb[4] = {xs0, xs1, xs2, xs3};
    auto issue = [&](auto jc, int i) {
        constexpr int j = decltype(jc)::value;
        const bool live = i < nr;  // uniform
        const int u = wave + kB2Waves * i;
#pragma unroll
        for (int r = 0; r < R; ++r)
            b2s_load<GS, FMT>(cp[j][r], sp[j][r], pr, sr, vo_code[r], vo_scale[r], u, live);
        b2s_stage_x(xsb[j] + wave * kB2sXBytes, xr, live ? xo_ld0 : kNoRecordOffset,
                    live ? xo_ld1 : kNoRecordOffset,
                    live ? uniform_offset((int64_t)u * kB2mRound * 2) : 0);
    };
    if (nr > 0) {
        issue(std::integral_constant<int, 0>{}, 0);
        issue(std::integral_constant<int, 1>{}, 1);
        issue(std::integral_constant<int, 2>{}, 2);
        issue(std::integral_constant<int, 3>{}, 3);
    }
    __syncthreads();  // selector table ready
    const char* lut = reinterpret_cast<const char*>(lut_storage) +
                      (FMT == kFmtTernary ? kLutBaseOffset : 0u);
    for (int i0 = 0; i0 < nr; i0 += 4) {  // uniform within the wave
        if (i0 + 4 < nr) {
            [&]<int... J>(std::integer_sequence<int, J...>) {
                (([&] {
                     vm_wait_le<3 * L>();  // slot J's round has landed; the other three may fly
                     if (i0 + J < nr)
                         B2mRound<DT, GS, FMT, R>::run(cp[J], sp[J], lut, slot, xsb[J], xo, acc);
                     lds_wait_all();  // this wave's reads of slot J's buffer are done
                     issue(std::integral_constant<int, J>{}, i0 + 4 + J);
                 })(),
                 ...);
            }(std::make_integer_sequence<int, 4>{});
        } else {
            // the last four slots: no refills (a spare load past the buffers' ends still
            // takes a memory round trip to return, which the wave's end would wait for)
            [&]<int... J>(std::integer_sequence<int, J...>) {
                (([&] {
                     vm_wait_le<(3 - J) * L>();
                     if (i0 + J < nr)
                         B2mRound<DT, GS, FMT, R>::run(cp[J], sp[J], lut, slot, xsb[J], xo, acc);
                 })(),
                 ...);
            }(std::make_integer_sequence<int, 4>{});
        }
    }
    vm_wait_all();  // every load has landed (the last pass waited for them all)

    // add the waves' partial sums (each wave's in its own part of buffer 0); lane (g, n)
    // holds rows m = 4g + q of column n
    f32x4* const red = reinterpret_cast<f32x4*>(xs0);
    constexpr int kRedWave = kB2sXBytes / 16;
#pragma unroll
    for (int r = 0; r < R; ++r) red[wave * kRedWave + r * 64 + lane] = acc[r];
    __syncthreads();
    if (wave != 0) return;
#pragma unroll
    for (int r = 0; r < R; ++r) {
#pragma unroll
        for (int w2 = 1; w2 < kB2Waves; ++w2) {
            const f32x4 o = red[w2 * kRedWave + r * 64 + lane];
            acc[r][0] += o[0];
            acc[r][1] += o[1];
            acc[r][2] += o[2];
            acc[r][3] += o[3];
        }
        const int64_t row = (tile * R + r) * 16 + i16;
        if (row < N) {
            const float bv = bias ? load_as_f32<DT>(bias, row) : 0.f;
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const int m = 4 * g + q;
                if (m < M)
                    store_from_f32<DT>(y, (int64_t)m * job.y_ld + job.y_col + row,
                                       acc[r][q] + bv + lora_term<DT>(lora, m, row));
            }
        }
    }
}


// ---- the B-operand GEMV at 4 < M <= 16 for K <= 4096: activations resident, every load issued first
//
// gemv2m_kernel stages each wave's 16 activation rows per 256-k round (8 KB of LDS per round
// for 1 KB of a tile's weights), so LDS limits it to two rounds in flight per wave and a
// per-linear launch pays several memory round trips.  Here a workgroup of 8 waves stages
// all 16 x K activations once (at most 128 KB: one workgroup per CU) for its TPW row tiles,
// and each wave requests the codes and scales of all of its rounds (u = w, w + 8: K is split
// over the 8 waves) for all TPW tiles into registers at its first instructions; the tiles
// share each A fragment read.  Rounds past K load past the buffers' ends (zeros, no memory
// traffic) and are not computed.  The activation stage is block b (round b, 8 KB) at 8 KB b
// in gemv2m_kernel's layout; wave w stages blocks w and w + 8; an explicit wait for those
// loads (the weights may still be in flight) and a plain barrier make them visible to
// every wave.  The 8 waves' partial sums of each tile meet in LDS.
constexpr int kB2xWaves = 8;
constexpr int kB2xMaxK = 4096;

template <int SLOTS>
__device__ __forceinline__ uint4 lut_item(int i, int kind);

__device__ __forceinline__ void b2x_stage_block(char* xb, __amdgpu_buffer_rsrc_t x,
                                                const uint32_t (&xo)[8], int so) {
#pragma unroll
    for (int q = 0; q < 8; ++q)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(x, lds_ptr(xb + 1024 * q), 16, xo[q], so, 0, 0);
}

template <int DT, int GS, int FMT, int TPW>
__global__ __launch_bounds__(64 * kB2xWaves) void gemv2x_kernel(GemvLaunch args) {
    int64_t wg = blockIdx.x;
    // the job as loaded (per-linear q/o at M = 16 measured 6.7 us against 7.1 with the
    // scalar copy, which the other kernels take)
    const GemvJob job = gemv_job_of<false>(args, wg);
    const void* const x = job.x ? job.x : args.x;
    void* const y = job.y ? job.y : args.y;
    const int M = args.M;
    const int64_t N = job.N, K = job.K;
    const LoraEp lora{job.lora_u, job.lora_b, job.lora_r,
                      job.lora_ldu ? job.lora_ldu : job.lora_r, job.N};
    static_assert(TPW == 1 || TPW == 2 || TPW == 4, "row tiles per workgroup");
    // formats whose decode table is computed, not read from memory (a load there would make
    // the table writes wait for every load issued before it)
    static_assert(FMT == kFmtTernary || FMT == kFmt2Bit, "ternary or 2-bit codes");
    constexpr int kBlocks = kB2xMaxK / kB2mRound;  // 16 rounds of 256 k
    constexpr int NR = kBlocks / kB2xWaves;       // rounds per wave
    constexpr int L = 2 * TPW;                    // loads per round: codes and scales per tile
    static_assert(NR * L < 64, "wait count range");
    __shared__ uint4 lut_storage[FMT == kFmtTernary ? kLutValidStorageU4 : kB2LutU4];
    __shared__ __attribute__((aligned(128))) char xs[kBlocks * kB2mXBytes];
    static_assert(kB2xWaves * TPW * 64 * 16 <= kBlocks * kB2mXBytes, "partial sums fit");

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int g = lane >> 4, i16 = lane & 15;
    const int T = (int)(K / kB2mRound);
    const uint32_t rowbytes = (uint32_t)(FMT == kFmtTernary ? K * 3 / 16 : K / 4);
    constexpr uint32_t kLaneBytes = FMT == kFmtTernary ? 12u : 16u;
    const uint32_t srowbytes = (uint32_t)(K * 2 / GS);
    const __amdgpu_buffer_rsrc_t pr = __builtin_amdgcn_make_buffer_rsrc(
        (void*)job.packed, (short)0, (int)(N * rowbytes), kRsrcWord3);
    const __amdgpu_buffer_rsrc_t sr = __builtin_amdgcn_make_buffer_rsrc(
        (void*)job.scales, (short)0, (int)(N * srowbytes), kRsrcWord3);
    const __amdgpu_buffer_rsrc_t xr = __builtin_amdgcn_make_buffer_rsrc(
        (void*)x, (short)0, (int)(M * K * 2), kRsrcWord3);

    // this wave's activation blocks first (every block is read by every wave of a round)
    uint32_t xo_ld[8];
#pragma unroll
    for (int q = 0; q < 8; ++q) xo_ld[q] = b2m_x_offset(q, lane, M, K);
#pragma unroll
    for (int i = 0; i < NR; ++i) {
        const int b = wave + kB2xWaves * i;
        uint32_t xo_b[8];
#pragma unroll
        for (int q = 0; q < 8; ++q) xo_b[q] = b < T ? xo_ld[q] : kNoRecordOffset;
        b2x_stage_block(xs + b * kB2mXBytes, xr, xo_b,
                        b < T ? uniform_offset((int64_t)b * kB2mRound * 2) : 0);
    }
    // then the codes and scales of its rounds of every tile (rows past N read zeros)
    uint32_t vo_code[TPW], vo_scale[TPW];
#pragma unroll
    for (int r = 0; r < TPW; ++r) {
        const uint32_t row = (uint32_t)((wg * TPW + r) * 16 + i16);
        vo_code[r] = row * rowbytes + kLaneBytes * g;
        vo_scale[r] = row * srowbytes + (128u / GS) * g;
    }
    uint4 cp[NR][TPW], sp[NR][TPW];
#pragma unroll
    for (int i = 0; i < NR; ++i) {
        const int u = wave + kB2xWaves * i;
#pragma unroll
        for (int r = 0; r < TPW; ++r)
            b2s_load<GS, FMT>(cp[i][r], sp[i][r], pr, sr, vo_code[r], vo_scale[r], u, u < T);
    }

    // decode table (computed) while the loads fly
    if constexpr (FMT == kFmtTernary) {
        for (int i = (int)threadIdx.x; i < kLutValidStorageU4; i += 64 * kB2xWaves)
            lut_storage[i] = lut_item<kLutSlots>(i, kLutMasks);
    } else {
        fill_b2sel<64 * kB2xWaves>(lut_storage);
    }
    // this wave's activation blocks have landed when at most its weight loads fly; the
    // plain barrier (no fence) leaves those in flight
    vm_wait_le<NR * L>();
    lds_wait_all();
    asm volatile("s_barrier" ::: "memory");

    const char* lut = reinterpret_cast<const char*>(lut_storage) +
                      (FMT == kFmtTernary ? kLutBaseOffset : 0u);
    const uint32_t slot = FMT == kFmtTernary ? (uint32_t)(lane & (kLutSlots - 1)) * 8u
                                             : (uint32_t)(lane & 31) * 4u;
    const uint32_t gu = (uint32_t)g, iu = (uint32_t)i16;
    const uint32_t xo =
        512u * iu + 16u * ((8u * gu & 16u) | ((8u * gu & 8u) ^ (iu & 8u)) | (iu & 7u));
    f32x4 acc[TPW];
#pragma unroll
    for (int r = 0; r < TPW; ++r) acc[r] = f32x4{0.f, 0.f, 0.f, 0.f};
    [&]<int... I>(std::integer_sequence<int, I...>) {
        (([&] {
             vm_wait_le<L * (NR - 1 - I)>();  // round I's code and scale loads have landed
             const int u = wave + kB2xWaves * I;
             if (u < T)
                 B2mRound<DT, GS, FMT, TPW>::run(cp[I], sp[I], lut, slot, xs + u * kB2mXBytes,
                                                 xo, acc);
         })(),
         ...);
    }(std::make_integer_sequence<int, NR>{});

    // every wave's partial sums of every tile through the (no longer read) stage; wave r <
    // TPW adds tile r's; lane (g, n) holds rows m = 4g + q of column n
    f32x4* const red = reinterpret_cast<f32x4*>(xs);
    __syncthreads();
#pragma unroll
    for (int r = 0; r < TPW; ++r) red[(wave * TPW + r) * 64 + lane] = acc[r];
    __syncthreads();
    if (wave >= TPW) return;
    f32x4 o = red[wave * 64 + lane];
#pragma unroll
    for (int w2 = 1; w2 < kB2xWaves; ++w2) {
        const f32x4 p = red[(w2 * TPW + wave) * 64 + lane];
        o[0] += p[0];
        o[1] += p[1];
        o[2] += p[2];
        o[3] += p[3];
    }
    const int64_t row = (wg * TPW + wave) * 16 + i16;
    if (row < N) {
        const float bv = job.bias ? load_as_f32<DT>(job.bias, row) : 0.f;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const int m = 4 * g + q;
            if (m < M)
                store_from_f32<DT>(y, (int64_t)m * job.y_ld + job.y_col + row,
                                   o[q] + bv + lora_term<DT>(lora, m, row));
        }
    }
}


// ---- the same for 4096 < K <= 16384 (down): weights prefetched, activations double-buffered per wave
//
// One row tile per workgroup of 8 waves; wave w takes the 256-k rounds u = w + 8 i, i < 8,
// requests the codes and scales of all of them into registers at its first instructions
// (rounds past K load past the buffers' ends: zeros, no traffic, issued with the others so
// that they add no round trip at the end), and stages the activations of its own rounds two
// ahead in its own two 8 KB buffers (the 16 activation rows come from L2), so that no wave
// reads another's stage and only the decode table needs a barrier.
constexpr int kB2xkRounds = 8;  // rounds per wave: K <= 8 * 8 * 256

template <int DT, int GS, int FMT>
__global__ __launch_bounds__(64 * kB2xWaves) void gemv2xk_kernel(GemvLaunch args) {
    int64_t wg = blockIdx.x;
    const GemvJob job = gemv_job_of(args, wg);
    const void* const x = job.x ? job.x : args.x;
    void* const y = job.y ? job.y : args.y;
    const int M = args.M;
    const int64_t N = job.N, K = job.K;
    const LoraEp lora{job.lora_u, job.lora_b, job.lora_r,
                      job.lora_ldu ? job.lora_ldu : job.lora_r, job.N};
    static_assert(FMT == kFmtTernary || FMT == kFmt2Bit, "ternary or 2-bit codes");
    constexpr int NR = kB2xkRounds;
    __shared__ uint4 lut_storage[FMT == kFmtTernary ? kLutValidStorageU4 : kB2LutU4];
    __shared__ __attribute__((aligned(128))) char xs0[kB2xWaves * kB2mXBytes];
    __shared__ __attribute__((aligned(128))) char xs1[kB2xWaves * kB2mXBytes];
    static_assert(kB2xWaves * 64 * 16 <= kB2xWaves * kB2mXBytes, "partial sums fit");

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int g = lane >> 4, i16 = lane & 15;
    const int T = (int)(K / kB2mRound);
    const int nr = wave < T ? (T - 1 - wave) / kB2xWaves + 1 : 0;  // this wave's rounds
    const uint32_t rowbytes = (uint32_t)(FMT == kFmtTernary ? K * 3 / 16 : K / 4);
    constexpr uint32_t kLaneBytes = FMT == kFmtTernary ? 12u : 16u;
    const uint32_t srowbytes = (uint32_t)(K * 2 / GS);
    const __amdgpu_buffer_rsrc_t pr = __builtin_amdgcn_make_buffer_rsrc(
        (void*)job.packed, (short)0, (int)(N * rowbytes), kRsrcWord3);
    const __amdgpu_buffer_rsrc_t sr = __builtin_amdgcn_make_buffer_rsrc(
        (void*)job.scales, (short)0, (int)(N * srowbytes), kRsrcWord3);
    const __amdgpu_buffer_rsrc_t xr = __builtin_amdgcn_make_buffer_rsrc(
        (void*)x, (short)0, (int)(M * K * 2), kRsrcWord3);
    uint32_t xo_ld[8];
#pragma unroll
    for (int q = 0; q < 8; ++q) xo_ld[q] = b2m_x_offset(q, lane, M, K);
    char* const xw0 = xs0 + wave * kB2mXBytes;
    char* const xw1 = xs1 + wave * kB2mXBytes;
    auto stage = [&](char* xw, int i) {  // activations of this wave's round i
        const int u = wave + kB2xWaves * i;
        uint32_t xo_b[8];
#pragma unroll
        for (int q = 0; q < 8; ++q) xo_b[q] = i < nr ? xo_ld[q] : kNoRecordOffset;
        b2x_stage_block(xw, xr, xo_b, i < nr ? uniform_offset((int64_t)u * kB2mRound * 2) : 0);
    };

    // round 0's activations, every round's codes and scales, round 1's activations
    stage(xw0, 0);
    const uint32_t row = (uint32_t)(wg * 16 + i16);  // rows past N read zeros
    const uint32_t vo_code = row * rowbytes + kLaneBytes * g;
    const uint32_t vo_scale = row * srowbytes + (128u / GS) * g;
    uint4 cp[NR], sp[NR];
#pragma unroll
    for (int i = 0; i < NR; ++i)
        b2s_load<GS, FMT>(cp[i], sp[i], pr, sr, vo_code, vo_scale, wave + kB2xWaves * i, i < nr);
    stage(xw1, 1);

    if constexpr (FMT == kFmtTernary) {
        for (int i = (int)threadIdx.x; i < kLutValidStorageU4; i += 64 * kB2xWaves)
            lut_storage[i] = lut_item<kLutSlots>(i, kLutMasks);
    } else {
        fill_b2sel<64 * kB2xWaves>(lut_storage);
    }
    lds_wait_all();
    asm volatile("s_barrier" ::: "memory");  // the table (the loads stay in flight)

    const char* lut = reinterpret_cast<const char*>(lut_storage) +
                      (FMT == kFmtTernary ? kLutBaseOffset : 0u);
    const uint32_t slot = FMT == kFmtTernary ? (uint32_t)(lane & (kLutSlots - 1)) * 8u
                                             : (uint32_t)(lane & 31) * 4u;
    const uint32_t gu = (uint32_t)g, iu = (uint32_t)i16;
    const uint32_t xo =
        512u * iu + 16u * ((8u * gu & 16u) | ((8u * gu & 8u) ^ (iu & 8u)) | (iu & 7u));
    f32x4 acc[1] = {f32x4{0.f, 0.f, 0.f, 0.f}};
    // round i: its activations have landed when at most the next round's (and, for round 0,
    // the weights') loads fly (none past the wave's last round); then its buffer takes round
    // i + 2 if there is one
    [&]<int... I>(std::integer_sequence<int, I...>) {
        (([&] {
             if (I < nr) {  // uniform
                 if constexpr (I == 0) vm_wait_le<2 * NR + 8>();
                 else if (I + 1 < nr) vm_wait_le<8>();
                 else vm_wait_all();
                 char* const xw = (I % 2) ? xw1 : xw0;
                 B2mRound<DT, GS, FMT, 1>::run(reinterpret_cast<const uint4(&)[1]>(cp[I]),
                                               reinterpret_cast<const uint4(&)[1]>(sp[I]), lut,
                                               slot, xw, xo, acc);
                 if constexpr (I + 2 < NR) {
                     if (I + 2 < nr) {
                         lds_wait_all();  // this wave's reads of the buffer are done
                         stage(xw, I + 2);
                     }
                 }
             }
         })(),
         ...);
    }(std::make_integer_sequence<int, NR>{});

    // the 8 waves' partial sums through the (no longer read) stage; lane (g, n) holds rows
    // m = 4g + q of column n
    f32x4* const red = reinterpret_cast<f32x4*>(xs0);
    __syncthreads();
    red[wave * 64 + lane] = acc[0];
    __syncthreads();
    if (wave != 0) return;
    f32x4 o = acc[0];
#pragma unroll
    for (int w2 = 1; w2 < kB2xWaves; ++w2) {
        const f32x4 p = red[w2 * 64 + lane];
        o[0] += p[0];
        o[1] += p[1];
        o[2] += p[2];
        o[3] += p[3];
    }
    if ((int64_t)row < N) {
        const float bv = job.bias ? load_as_f32<DT>(job.bias, row) : 0.f;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const int m = 4 * g + q;
            if (m < M)
                store_from_f32<DT>(y, (int64_t)m * job.y_ld + job.y_col + row,
                                   o[q] + bv + lora_term<DT>(lora, m, row));
        }
    }
}


// ------------------------------------------------------------------------- staged-tile GEMV
//
// Decode GEMV (M <= 4) for launches with few row tiles: the per-linear launches of a
// decoder's linears (1-15 MB each).  Such a launch never streams long enough to reach the
// HBM ceiling; its time is the kernel start, one memory round trip and the work that depends
// on it.  So every wave issues all of its loads at its first instructions: the codes and
// scales of its own 1024-k rounds of the workgroup's 16-row tile and the matching
// activations, by 16-byte buffer->LDS loads into the wave's own stage (the 224 per-linear
// launches of the 32-layer stack move these bytes in about 0.7 ms on MI355X, against 0.68 ms
// for a plain read of the weights).  The decode table is computed while they are in flight
// (one workgroup barrier); then each wave waits only for its own loads, round by round, and
// runs that round's MFMAs while its later rounds still arrive.
//
// Work: one workgroup of 4 waves per 16-row tile; wave w takes rounds [w U, min(w U + U, T))
// of the T = K / 1024 rounds.  In round u lane (g, n) holds codes 32g .. 32g + 31 of row n
// (k = 1024u + 256g .. + 255) and their 8 group scales; step j (0..31) contracts
// k = 1024u + 256g + 8j + (0..7) with A row i16 = activation row i16 (lanes of rows >= M
// skip the read and keep zeros: only M lanes per lane group touch LDS) and B = code j's
// weights (table masks AND-ed with the scale word, as the other B-operand GEMVs).  Two
// accumulators alternate between steps; the waves' partial sums are added through LDS and
// wave 0 stores rows m < M.
//
// Stage of one round (each lane of a buffer->LDS load writes a fixed 16-byte slot, so the
// placement is chosen through the piece each lane fetches): codes, row n's 12 pieces at
// slots 12n + (p + n/4) mod 12; scales at group size 32, row n's 4 pieces at 4n + (p + n/4)
// mod 4 (group size 16: 8 pieces at 8n + (p + n/2) mod 8; group size 64: 2 pieces at
// 2n + (p + n/8) mod 2); then MM activation rows of 128 pieces, piece p of row m at
// m * 128 + (p ^ m).  The 16 lanes of a lane group then read 16 distinct bank groups.

constexpr int kTileWaves = 4;
constexpr uint32_t kTileRoundCodes = 16 * 192;  // one round's codes of 16 rows

// Scale bytes of one round of one 16-row tile at group size gs (1024 k per row: 2048 / gs
// bytes), in whole 1-KB loads: 2 KB at group size 16, 1 KB at 32, 1 KB at 64 (half used).
__host__ __device__ constexpr uint32_t tile_scale_region(int gs) { return gs == 16 ? 2048u : 1024u; }

// One wave's stage of one round for RT row tiles: the tiles' codes, their scales, then the
// activations (shared by the tiles).
template <int MM, int RT, int GS>
struct TileStage {
    static_assert(GS == 16 || GS == 32 || GS == 64, "group size 16, 32 or 64");
    static constexpr uint32_t kScaleRegion = tile_scale_region(GS);
    static constexpr uint32_t kScales = RT * kTileRoundCodes;     // offset of the scales
    static constexpr uint32_t kX = kScales + RT * kScaleRegion;   // offset of the activations
    static constexpr int kXLoads = (145 * (MM - 1) + 140 + 63) / 64;  // 1-KB loads of them
    static constexpr uint32_t kBytes = kX + kXLoads * 1024;           // one round
    static constexpr int kLoads = (3 + (int)kScaleRegion / 1024) * RT + kXLoads;  // per round
};

// One 16-byte-per-lane buffer->LDS load (1 KB per wave) into `dst`.  (Not a template: the
// host pass drops a kernel template that calls this builtin directly.)
__device__ __forceinline__ void dma_1k(__amdgpu_buffer_rsrc_t r, char* dst, uint32_t voffset) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, lds_ptr(dst), 16, voffset, 0, 0, 0);
}

// Issues round u's loads into `stg`: for each of the rt row tiles (rows row0 + 16 r) three
// of codes and the scales (group size gs: one load, two at 16), then `xloads` of
// activations.
__device__ __forceinline__ void tile_issue(char* stg, __amdgpu_buffer_rsrc_t pr,
                                           __amdgpu_buffer_rsrc_t sr, __amdgpu_buffer_rsrc_t xr,
                                           uint32_t row0, uint32_t rowbytes, uint32_t srowbytes,
                                           uint32_t xrowbytes, int u, int lane, int xloads,
                                           int M, int rt, int gs) {
    for (int r = 0; r < rt; ++r) {
#pragma unroll
        for (int t = 0; t < 3; ++t) {
            const uint32_t sl = 64u * t + lane, n = sl / 12u, q = sl - 12u * n;
            const uint32_t p = (q + 12u - n / 4u) % 12u;
            dma_1k(pr, stg + kTileRoundCodes * r + 1024 * t,
                   (row0 + 16u * r + n) * rowbytes + 192u * u + 16u * p);
        }
    }
    const uint32_t sreg = tile_scale_region(gs);
    for (int r = 0; r < rt; ++r) {
        char* const sdst = stg + kTileRoundCodes * rt + sreg * r;
        if (gs == 32) {
            const uint32_t n = (uint32_t)lane >> 2, q = (uint32_t)lane & 3u;
            const uint32_t p = (q + 4u - (n / 4u) % 4u) % 4u;
            dma_1k(sr, sdst, (row0 + 16u * r + n) * srowbytes + 64u * u + 16u * p);
        } else if (gs == 16) {
            for (int h = 0; h < 2; ++h) {
                const uint32_t n = 8u * h + ((uint32_t)lane >> 3), q = (uint32_t)lane & 7u;
                const uint32_t p = (q - (n >> 1)) & 7u;
                dma_1k(sr, sdst + 1024 * h, (row0 + 16u * r + n) * srowbytes + 128u * u + 16u * p);
            }
        } else {  // 64: 16 rows x 32 bytes from lanes 0..31; the others read zeros
            const uint32_t n = ((uint32_t)lane >> 1) & 15u, q = (uint32_t)lane & 1u;
            const uint32_t p = (q - (n >> 3)) & 1u;
            dma_1k(sr, sdst, lane < 32 ? (row0 + 16u * r + n) * srowbytes + 32u * u + 16u * p
                                       : 0xFFFFFFF0u);
        }
    }
    // activations: row m's piece p at slot 145 m + p + 4 (p / 32) (the lane groups' 32-piece
    // runs 36 slots apart); unused slots and rows >= M read zeros
    for (int i = 0; i < xloads; ++i) {
        const uint32_t sl = 64u * i + lane, m = sl / 145u, r = sl - 145u * m;
        const uint32_t blk = r / 36u, wi = r - 36u * blk;
        const uint32_t off = (m < (uint32_t)M && blk < 4u && wi < 32u)
                                 ? m * xrowbytes + 2048u * u + 16u * (32u * blk + wi)
                                 : 0xFFFFFFF0u;
        dma_1k(xr, stg + (kTileRoundCodes + sreg) * rt + 1024 * i, off);
    }
}

// Depth of the software pipeline of a round: the table and activation reads of step
// J + kTileAhead are issued before the MFMA of step J (with one wave per SIMD, a step that
// waited for its own reads would expose the whole LDS latency).
constexpr int kTileAhead = 4;

// The staged-tile kernel's table: 32 slices (conflict-free b64 reads: 2.2 clk per wave
// read on MI355X against 3.7 with 16 slices, where neighbouring lanes share banks), holding
// the coordinates themselves (+-1, 0 in the activation dtype); 16 slices where two row tiles
// per wave need the LDS for their stages.
template <int RT> constexpr int tile_slots() { return RT == 1 ? 32 : 16; }

// One post-scaled 1024-k round (the layout of gemv_ps_kernel): A row 4g' + m carries
// activation row m only in lane group g''s k slots (every other lane's fragment is zero), so
// lane (g', n)'s MFMA result rows 4g' + q are the partial sums of its own codes for
// activation rows q; after the 4 steps of one scale group they are multiplied by that
// group's scale into the fp32 accumulators.  The table and activation reads of step
// J + kTileAhead are issued before the MFMA of step J; two D registers alternate between
// scale groups.
template <int DT, int MM, int RT, int GS>
struct TileRound {
    using G = LutGeom<tile_slots<RT>()>;
    static constexpr int kSpg = GS / 8;   // steps per scale group
    uint32_t cd[RT][12];  // this lane's 32 codes of each row tile
    uint32_t scw[RT][128 / GS];  // their 256 / GS group scales (fp16 pairs)
    const char* lut;
    const char* xa;   // this lane's A fragment of step 0 (activations or a zero run)
    uint32_t slot;

    struct Pending {
        uint4 a[kTileAhead], b[kTileAhead][RT];
    };

    template <int J>
    __device__ __forceinline__ void reads(Pending& p) const {
        constexpr int r = J % kTileAhead;
        p.a[r] = *reinterpret_cast<const uint4*>(xa + 16 * J);
#pragma unroll
        for (int t = 0; t < RT; ++t) {
            const uint32_t d[3] = {cd[t][3 * (J / 8)], cd[t][3 * (J / 8) + 1],
                                   cd[t][3 * (J / 8) + 2]};
            const uint32_t z = code_z<J % 8, G::kCodeShift>(d, slot);
            const uint32_t h = __umulhi(z, G::kHiMagic);
            const uint2 ml = *reinterpret_cast<const uint2*>(lut + lo_addr_of<G::kStride>(h, z));
            const uint2 mh = *reinterpret_cast<const uint2*>(lut + (h * G::kStride + slot));
            p.b[r][t] = make_uint4(ml.x, ml.y, mh.x, mh.y);
        }
    }
    template <int J>
    __device__ __forceinline__ void step(Pending& p, f32x4 (&d)[2][RT],
                                         float (&acc)[RT][MM]) const {
        constexpr int r = J % kTileAhead, gi = J / kSpg;  // scale group of the step
        const uint4 a = p.a[r];
        uint4 b[RT];
#pragma unroll
        for (int t = 0; t < RT; ++t) b[t] = p.b[r][t];
        if constexpr (J + kTileAhead < 32) reads<(J + kTileAhead < 32 ? J + kTileAhead : 0)>(p);
#pragma unroll
        for (int t = 0; t < RT; ++t) {
            f32x4& dg = d[gi & 1][t];
            dg = mfma16<DT>(a, b[t], J % kSpg == 0 ? f32x4{0.f, 0.f, 0.f, 0.f} : dg);
        }
        if constexpr (J % kSpg == kSpg - 1) {  // scale group gi complete: post-scale it
#pragma unroll
            for (int t = 0; t < RT; ++t) {
                f32x4& dg = d[gi & 1][t];
                float s0, s1;
                scale_pair_f32<DT>(scw[t][gi / 2], s0, s1);
                const float sg = (gi & 1) ? s1 : s0;
#pragma unroll
                for (int q = 0; q < MM; ++q) acc[t][q] = __builtin_fmaf(dg[q], sg, acc[t][q]);
                keep_mfma_result(dg, acc[t][0]);
            }
        }
    }
    template <int... J>
    __device__ __forceinline__ void prologue(Pending& p, std::integer_sequence<int, J...>) const {
        (reads<J>(p), ...);
    }
    template <int... J>
    __device__ __forceinline__ void steps(float (&acc)[RT][MM], std::integer_sequence<int, J...>) const {
        Pending p;
        f32x4 d[2][RT];
        prologue(p, std::make_integer_sequence<int, kTileAhead>{});
        (step<J>(p, d, acc), ...);
    }
};

// 16-byte item i of a bank-sliced table of `kind` (e8t_lut.h) with SLOTS slices, computed:
// two slices of entry i / (SLOTS / 2) - guard (the guard entry is zero).
template <int SLOTS>
__device__ __forceinline__ uint4 lut_item(int i, int kind) {
    const int e = i / (SLOTS / 2) - LutGeom<SLOTS>::kGuard;
    if (e < 0) return make_uint4(0u, 0u, 0u, 0u);
    const int d0 = e % 3, d1 = (e / 3) % 3, d2 = (e / 9) % 3, d3 = (e / 27) % 3;
    const uint32_t w0 = lut_half(kind, d0) | (lut_half(kind, d1) << 16);
    const uint32_t w1 = lut_half(kind, d2) | (lut_half(kind, d3) << 16);
    return make_uint4(w0, w1, w0, w1);
}


// ---- LoRA down-projection inside the staged-tile launch (one round per wave, rank 8)
//
// The fused epilogue adds u @ B with u = scaling * (x @ A) [M, 8] (lattice.py:839-842).
// Instead of a separate down-projection launch before the GEMV, every workgroup of an
// adapter job forms u itself: each wave adds the k range of its own round.  Lane l takes
// k = 16 l .. 16 l + 15 of the round: 16 rows of A (16 bytes each) and two 16-byte
// activation pieces per row m, loaded into registers before the round's weights are
// requested, so that the v_dot2 products of k pairs (the pair of A values of one column is
// put together by one v_perm) and the lanes' sum run while the weights are in flight.  The
// waves' totals meet in LDS, and the epilogue lanes read u there.
constexpr int kLoraInlineRank = 8;
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));

template <int DT>
__device__ __forceinline__ float dot2_acc(uint32_t a, uint32_t b, float c) {
    if constexpr (DT == kBF16)
        return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, a),
                                               __builtin_bit_cast(bf16x2_t, b), c, false);
    else
        return __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2_t, a),
                                      __builtin_bit_cast(f16x2_t, b), c, false);
}

// Rows k0 + 16 lane .. + 15 of A [K, 8] (16-byte rows), through buffer (not flat) loads: a
// flat load could read LDS, so the compiler would first wait for every pending
// buffer->LDS load of the stage.
__device__ __forceinline__ void lora_load_a(const void* a, int64_t K, int64_t k0, int lane,
                                            uint4 (&ar)[16]) {
    const __amdgpu_buffer_rsrc_t r = __builtin_amdgcn_make_buffer_rsrc(
        (void*)a, (short)0, (int)(K * 2 * kLoraInlineRank), kRsrcWord3);
    const uint32_t vo = (uint32_t)(k0 + 16 * lane) * 16u;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(r, vo + 16u * i, 0, 0);
        ar[i] = make_uint4(v.x, v.y, v.z, v.w);
    }
}

// B[j][row] for j < 8 (bf16/fp16 bits), from a buffer of `live` columns (0: zeros).
__device__ __forceinline__ void lora_load_bcol(const void* b, int64_t live, int64_t N,
                                               int64_t row, uint32_t (&bq)[kLoraInlineRank]) {
    const __amdgpu_buffer_rsrc_t r = __builtin_amdgcn_make_buffer_rsrc(
        (void*)b, (short)0, (int)(live * kLoraInlineRank * 2), kRsrcWord3);
#pragma unroll
    for (int j = 0; j < kLoraInlineRank; ++j)
        bq[j] = __builtin_amdgcn_raw_buffer_load_b16(r, (uint32_t)(j * N + row) * 2u, 0, 0);
}

// x[m][k0 + 16 lane .. + 15] for m < MM as two 16-byte pieces per row (rows >= M lie past
// the buffer's M * K * 2 bytes and read zeros).
template <int MM>
__device__ __forceinline__ void lora_load_x(const void* x, int M, int64_t K, int64_t k0,
                                            int lane, uint4 (&xr)[2 * MM]) {
    const __amdgpu_buffer_rsrc_t r = __builtin_amdgcn_make_buffer_rsrc(
        (void*)x, (short)0, (int)(M * K * 2), kRsrcWord3);
#pragma unroll
    for (int m = 0; m < MM; ++m) {
        const uint32_t vo = (uint32_t)((int64_t)m * K + k0 + 16 * lane) * 2u;
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(r, vo + 16u * h, 0, 0);
            xr[2 * m + h] = make_uint4(v.x, v.y, v.z, v.w);
        }
    }
}

// part[m][j] = sum over this lane's 16 k of x[m][k] A[k][j].
template <int DT, int MM>
__device__ __forceinline__ void lora_lane_part(const uint4 (&ar)[16], const uint4 (&xr)[2 * MM],
                                               float (&part)[MM][kLoraInlineRank]) {
    uint32_t lo[8][4], hi[8][4];  // (A[k][c], A[k + 1][c]) for k pair kp, columns 2h, 2h + 1
#pragma unroll
    for (int kp = 0; kp < 8; ++kp) {
        const uint32_t r0[4] = {ar[2 * kp].x, ar[2 * kp].y, ar[2 * kp].z, ar[2 * kp].w};
        const uint32_t r1[4] = {ar[2 * kp + 1].x, ar[2 * kp + 1].y, ar[2 * kp + 1].z,
                                ar[2 * kp + 1].w};
#pragma unroll
        for (int h = 0; h < 4; ++h) {
            lo[kp][h] = __builtin_amdgcn_perm(r1[h], r0[h], 0x05040100u);
            hi[kp][h] = __builtin_amdgcn_perm(r1[h], r0[h], 0x07060302u);
        }
    }
#pragma unroll
    for (int m = 0; m < MM; ++m) {
        const uint4 x0 = xr[2 * m], x1 = xr[2 * m + 1];
        const uint32_t xw[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
#pragma unroll
        for (int j = 0; j < kLoraInlineRank; ++j) part[m][j] = 0.f;
#pragma unroll
        for (int kp = 0; kp < 8; ++kp)
#pragma unroll
            for (int h = 0; h < 4; ++h) {
                part[m][2 * h] = dot2_acc<DT>(xw[kp], lo[kp][h], part[m][2 * h]);
                part[m][2 * h + 1] = dot2_acc<DT>(xw[kp], hi[kp][h], part[m][2 * h + 1]);
            }
    }
}

// One halving exchange of wave_sum_scatter at offset 32 >> ST over the first 2h values, with
// every index a compile-time constant (a select between array elements indexed by a loop
// variable becomes a dynamically indexed private array).
template <int h, int o, int... I>
__device__ __forceinline__ void halve_exchange(float* w, bool up, std::integer_sequence<int, I...>) {
    ((w[I] = (up ? w[I + h] : w[I]) + __shfl_xor(up ? w[I] : w[I + h], o)), ...);
}

// Sum of v[c] over the wave's 64 lanes for each of its V values (V a power of two <= 64),
// by halving exchanges: at offset o = 32, 16, ... a lane keeps the upper half of its live
// values if lane & o, sends the other half to lane ^ o and adds what it receives; then the
// lanes holding the same value add theirs.  Lane l returns the total of value l >> (6 - log2 V).
template <int V>
__device__ __forceinline__ float wave_sum_scatter(const float (&v)[V], int lane) {
    constexpr int LV = V == 1 ? 0 : V == 2 ? 1 : V == 4 ? 2 : V == 8 ? 3 : V == 16 ? 4 : V == 32 ? 5 : 6;
    static_assert((1 << LV) == V, "V is a power of two <= 64");
    float w[V];
    [&]<int... I>(std::integer_sequence<int, I...>) { ((w[I] = v[I]), ...); }(
        std::make_integer_sequence<int, V>{});
    [&]<int... ST>(std::integer_sequence<int, ST...>) {
        ((halve_exchange<(V >> ST) / 2, (32 >> ST)>(w, (lane & (32 >> ST)) != 0,
                                                    std::make_integer_sequence<int, (V >> ST) / 2>{})),
         ...);
    }(std::make_integer_sequence<int, LV>{});
    float t = w[0];
#pragma unroll
    for (int o = 32 >> LV; o >= 1; o >>= 1) t += __shfl_xor(t, o);
    return t;
}

// RT: row tiles per wave (they share the activation stage and the A fragment reads); a
// workgroup covers TPW * RT row tiles.
// TW: waves per row tile (the tile's K / 1024 rounds are spread over them, U each).
// LI: the launch forms LoRA u inside (args.lora_inline); a separate instantiation, since its
// adapter loads are issued on every wave of the launch.
template <int DT, int MM, int U, int TPW, int RT, int TW, int GS, bool LI = false>
__global__ __launch_bounds__(64 * TW * TPW)
__attribute__((amdgpu_waves_per_eu(RT == 2 ? 2 : 1))) void gemv_tile_kernel(GemvLaunch args) {
    using S = TileStage<MM, RT, GS>;
    constexpr int SL = tile_slots<RT>();
    using TileLut = LutGeom<SL>;
    constexpr int L = S::kLoads;
    constexpr int NW = TW * TPW;  // waves of the workgroup
    static_assert(L * U <= 63, "loads in flight per wave");
    __shared__ __attribute__((aligned(16))) char stage[NW * U * S::kBytes];
    __shared__ uint4 lut_storage[TileLut::kValidStorageU4];
    // zero A fragments: lane l of step J reads zrun[l + J] (distinct addresses, no broadcast)
    __shared__ uint4 zrun[96];
    // in-launch LoRA down-projection (the instantiation with one round per wave of 4, one
    // tile per wave and workgroup; elsewhere the extra registers would cost occupancy):
    // each wave's total of x @ A over its round
    constexpr bool kLoraIn = LI && U == 1 && RT == 1 && TPW == 1 && TW == kTileWaves;
    __shared__ float lora_tot[kLoraIn ? TW : 1][MM * kLoraInlineRank];

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
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int sub = wave / TW, wt = wave % TW;  // tile of the workgroup, K part
    const int64_t tile = ((wg - job.wg_begin) * TPW + sub) * RT;  // the wave's first tile
    const void* xbase = job.x ? job.x : args.x;
    void* ybase = job.y ? job.y : args.y;

    const int lane = threadIdx.x & 63;
    const int g = lane >> 4, i16 = lane & 15;
    const int64_t N = job.N, K = job.K;
    const int M = args.M;
    const int T = (int)(K / 1024);
    const uint32_t rowbytes = (uint32_t)(K * 3 / 16), srowbytes = (uint32_t)(K * 2 / GS);
    const uint32_t row0 = (uint32_t)(tile * 16);
    const int u0 = wt * U;
    const int nr = T - u0 < U ? (T - u0 > 0 ? T - u0 : 0) : U;  // rounds of this wave

    // ---- every load first (rows >= N and activation rows >= M read zeros)
    // The in-launch adapter issues every load on every wave, with no branch, so that the
    // compiler's wait for the adapter's registers counts the stage loads issued after them
    // (a branch would make it wait for all of them); loads a wave does not need go to empty
    // buffers, which return zeros without a memory access.
    const bool dead = kLoraIn && nr == 0;  // a wave without a round (K < 4096)
    const __amdgpu_buffer_rsrc_t pr = __builtin_amdgcn_make_buffer_rsrc(
        (void*)job.packed, (short)0, dead ? 0 : (int)(N * rowbytes), kRsrcWord3);
    const __amdgpu_buffer_rsrc_t sr = __builtin_amdgcn_make_buffer_rsrc(
        (void*)job.scales, (short)0, dead ? 0 : (int)(N * srowbytes), kRsrcWord3);
    const __amdgpu_buffer_rsrc_t xr = __builtin_amdgcn_make_buffer_rsrc(
        (void*)xbase, (short)0, dead ? 0 : (int)(M * K * 2), kRsrcWord3);
    char* const wstage = stage + wave * U * S::kBytes;
    // the adapter's operands first (x and A of this wave's round, into registers; the
    // epilogue lanes' column of B, rows past N reading row N - 1), so that u is formed
    // while the weights are in flight
    const bool lora_in = kLoraIn && args.lora_inline && job.lora_r > 0;  // uniform
    const bool lora_wave = lora_in && nr > 0;
    uint4 lora_a[kLoraIn ? 16 : 1], lora_x[kLoraIn ? 2 * MM : 1];
    uint32_t lora_bq[kLoraIn ? kLoraInlineRank : 1];
    if constexpr (kLoraIn) {
        const int64_t k0 = (int64_t)u0 * 1024;
        lora_load_x<MM>(xbase, lora_wave ? M : 0, K, k0, lane, lora_x);
        lora_load_a(job.lora_a, lora_wave ? K : 0, k0, lane, lora_a);
        lora_load_bcol(job.lora_b, lora_in && wt == 0 ? N : 0, N,
                       (int64_t)row0 + i16 < N ? (int64_t)row0 + i16 : N - 1, lora_bq);
    }
#pragma unroll
    for (int i = 0; i < U; ++i)
        if (kLoraIn || i < nr)
            tile_issue(wstage + i * S::kBytes, pr, sr, xr, row0, rowbytes, srowbytes,
                       (uint32_t)(K * 2), u0 + i, lane, S::kXLoads, M, RT, GS);

    // ---- decode table (computed) while the loads are in flight
    for (int i = (int)threadIdx.x; i < TileLut::kValidStorageU4; i += 64 * NW)
        lut_storage[i] = lut_item<SL>(i, lut_values_kind<DT>());
    if (threadIdx.x < 96) zrun[threadIdx.x] = make_uint4(0u, 0u, 0u, 0u);

    // this wave's total of x @ A over its round (lanes 2c, 2c + 1 hold column c = 8 m + j;
    // lanes 8c .. 8c + 7 at M = 1) while the stage's loads are in flight: before the
    // barrier, which waits for every load of the wave
    if constexpr (kLoraIn) {
        if (lora_in) {
            constexpr int V = MM * kLoraInlineRank;
            float part[MM][kLoraInlineRank];
            if (lora_wave) {
                lora_lane_part<DT, MM>(lora_a, lora_x, part);
            } else {
#pragma unroll
                for (int m = 0; m < MM; ++m)
#pragma unroll
                    for (int j = 0; j < kLoraInlineRank; ++j) part[m][j] = 0.f;
            }
            const float v = wave_sum_scatter<V>(reinterpret_cast<const float(&)[V]>(part), lane);
            if ((lane & (64 / V - 1)) == 0) lora_tot[wt][lane / (64 / V)] = v;
        }
    }

    uint32_t bias_bits[RT];
#pragma unroll
    for (int t = 0; t < RT; ++t) {
        bias_bits[t] = 0u;
        if (wt == 0 && job.bias) {
            const int64_t r0 = (int64_t)row0 + 16 * t + i16;
            bias_bits[t] = ((const __attribute__((address_space(1))) uint16_t*)job.bias)[r0 < N ? r0 : N - 1];
        }
    }
    __syncthreads();

    const char* lut = reinterpret_cast<const char*>(lut_storage) + TileLut::kBaseOffset;
    const uint32_t slot = (uint32_t)(lane & (SL - 1)) * 8u;
    // A row i16 = 4g' + m is live in lane group g' for activation rows m < M: piece 32g + J of
    // row m (slot 145 m + 36 g + J); every other lane reads zeros
    const int am = i16 & 3;
    const bool a_live = (i16 >> 2) == g && am < M;
    const char* const zbase = reinterpret_cast<const char*>(zrun) + 16 * lane;
    const uint32_t xa0 = 16u * (145u * (uint32_t)am + 36u * (uint32_t)g);
    const uint32_t rq = (uint32_t)i16 / 4u;
    float acc[RT][MM];
#pragma unroll
    for (int t = 0; t < RT; ++t)
#pragma unroll
        for (int q = 0; q < MM; ++q) acc[t][q] = 0.f;
    auto round = [&](auto ic) {
        constexpr int i = decltype(ic)::value;
        if (i >= nr) return;
        // round i's loads have landed when at most the later rounds' are outstanding
        if (nr == U) vm_wait_le<L * (U - 1 - i)>();
        else vm_wait_all();
        const char* stg = wstage + i * S::kBytes;
        TileRound<DT, MM, RT, GS> r;
#pragma unroll
        for (int tt = 0; tt < RT; ++tt) {
#pragma unroll
            for (int t = 0; t < 3; ++t) {
                const uint32_t q = (3u * (uint32_t)g + (uint32_t)t + rq) % 12u;
                const uint4 v = *reinterpret_cast<const uint4*>(stg + kTileRoundCodes * tt +
                                                                (12u * i16 + q) * 16u);
                r.cd[tt][4 * t] = v.x;
                r.cd[tt][4 * t + 1] = v.y;
                r.cd[tt][4 * t + 2] = v.z;
                r.cd[tt][4 * t + 3] = v.w;
            }
            // this lane's scales: the 2048 / GS bytes of its 256 k (GS 16: pieces 2g, 2g + 1;
            // GS 32: piece g; GS 64: half g & 1 of piece g / 2)
            const char* const sreg = stg + S::kScales + S::kScaleRegion * tt;
            if constexpr (GS == 32) {
                const uint4 sc = *reinterpret_cast<const uint4*>(
                    sreg + (4u * i16 + (((uint32_t)g + rq) & 3u)) * 16u);
                r.scw[tt][0] = sc.x;
                r.scw[tt][1] = sc.y;
                r.scw[tt][2] = sc.z;
                r.scw[tt][3] = sc.w;
            } else if constexpr (GS == 16) {
#pragma unroll
                for (int h = 0; h < 2; ++h) {
                    const uint32_t pos = (2u * (uint32_t)g + h + ((uint32_t)i16 >> 1)) & 7u;
                    const uint4 sc = *reinterpret_cast<const uint4*>(sreg + 128u * i16 + 16u * pos);
                    r.scw[tt][4 * h] = sc.x;
                    r.scw[tt][4 * h + 1] = sc.y;
                    r.scw[tt][4 * h + 2] = sc.z;
                    r.scw[tt][4 * h + 3] = sc.w;
                }
            } else {
                const uint32_t pos = (((uint32_t)g >> 1) + ((uint32_t)i16 >> 3)) & 1u;
                const uint2 sc = *reinterpret_cast<const uint2*>(
                    sreg + 32u * i16 + 16u * pos + 8u * ((uint32_t)g & 1u));
                r.scw[tt][0] = sc.x;
                r.scw[tt][1] = sc.y;
            }
        }
        r.lut = lut;
        r.xa = a_live ? stg + S::kX + xa0 : zbase;
        r.slot = slot;
        r.steps(acc, std::make_integer_sequence<int, 32>{});
    };
    [&]<int... I>(std::integer_sequence<int, I...>) {
        (round(std::integral_constant<int, I>{}), ...);
    }(std::make_integer_sequence<int, U>{});
    // sum the four lane groups of each row (lane group q keeps activation row q), then the
    // waves through LDS (zrun is no longer read)
    float out[RT];
#pragma unroll
    for (int t = 0; t < RT; ++t) {
        out[t] = 0.f;
#pragma unroll
        for (int q = 0; q < MM; ++q) {
            float v = acc[t][q];
            v += __shfl_xor(v, 16);
            v += __shfl_xor(v, 32);
            if (q == g) out[t] = v;
        }
    }
    __syncthreads();
    // the waves' partial sums, in the stage (every wave has waited for all of its loads and
    // read its stage before the barrier)
    float* red = reinterpret_cast<float*>(stage);  // NW x RT x 64 floats
#pragma unroll
    for (int t = 0; t < RT; ++t) red[(wave * RT + t) * 64 + lane] = out[t];
    __syncthreads();
    if (wt != 0) return;
#pragma unroll
    for (int t = 0; t < RT; ++t) {
#pragma unroll
        for (int w2 = 1; w2 < TW; ++w2) out[t] += red[((wave + w2) * RT + t) * 64 + lane];
        const int64_t row = (int64_t)row0 + 16 * t + i16;
        if (g < M && row < N) {
            const float bv = job.bias ? bias_bits_to_f32<DT>(bias_bits[t]) : 0.f;
            float lt = 0.f;
            if (lora_in) {  // u[g][j] from the waves' totals, then u[g] . B[:, row]
#pragma unroll
                for (int j = 0; j < kLoraInlineRank; ++j) {
                    float uj = 0.f;
#pragma unroll
                    for (int w2 = 0; w2 < TW; ++w2) uj += lora_tot[kLoraIn ? w2 : 0][8 * g + j];
                    lt = __builtin_fmaf(job.lora_scaling * uj,
                                        bias_bits_to_f32<DT>(lora_bq[kLoraIn ? j : 0]), lt);
                }
            } else {
                lt = job_lora<DT>(job, g, row);
            }
            store_from_f32<DT>(ybase, (int64_t)g * job.y_ld + job.y_col + row, out[t] + bv + lt);
        }
    }
}

// ------------------------------------------------------------------------- host side

bool gemv_shape_ok(int64_t N, int64_t K) {
    // buffer offsets and record counts are 32-bit: every byte offset of the layer (plus
    // the row padding of the last tile set) must stay below 2^31
    return N >= 1 && K >= kChunk && K % kChunk == 0 && (N + 512) * (K * 3 / 16) < (1ll << 31) &&
           16 * K * 2 < (1ll << 31);
}

bool gemv_supported(const void* x, const uint8_t* packed, const uint16_t* scales, const void* y,
                    int64_t M, int64_t N, int64_t K, int64_t gs, int dt) {
    if (dt != kBF16 && dt != kF16) return false;
    if (gs != 32 || M < 1 || M > 16 || !gemv_shape_ok(N, K)) return false;
    if (((uintptr_t)x & 15u) || ((uintptr_t)packed & 3u) || ((uintptr_t)scales & 3u) ||
        ((uintptr_t)y & 1u))
        return false;
    return true;
}

GemvPlan gemv_pick(int64_t total_tiles, int64_t M) {
    GemvPlan p{};
    if (total_tiles >= 1024) {
        // enough row tiles to fill the GPU with one tile set per wave: streaming kernel
        p.wide = true;
        p.S = 1;
        // M <= 4: post-scaled kernel (mmax 1 or 4); otherwise the mask kernel
        p.mmax = M == 1 ? 1 : (M <= 4 ? 4 : 16);
        p.R = p.mmax == 16 ? 2 : (p.mmax == 4 && total_tiles < kPsOneTileBelow ? 1 : kPsTiles);
        // post-scaled kernel: consecutive tile groups per workgroup
        p.C = p.mmax == 16 ? 1 : kPsChunk;
        // waves sharing one table copy and one activation stage
        p.W = p.mmax == 16 ? kMaskWaves : (p.mmax == 4 && p.R == kPsTiles ? kPsWavesM4 : kPsWaves);
    } else if (M <= 4) {
        // small layers, M <= 4: one tile per workgroup, rounds split over its waves
        p.wide = false;
        p.split_ps = true;
        p.C = 1;
        p.R = 1;
        p.S = 1;
        p.W = 4;
        p.mmax = M == 1 ? 1 : 4;
    } else {
        // small layers: split K inside the workgroup to get enough waves
        p.wide = false;
        p.C = 1;
        p.R = 1;
        p.S = total_tiles >= 512 ? 2 : 4;
        p.W = 4;
        p.mmax = 16;
    }
    return p;
}

int64_t gemv_wgs_for(int64_t N, const GemvPlan& p) {
    const int64_t tiles = (N + 15) / 16;
    const int64_t per_wg = p.tile     ? p.tpw
                           : p.split_ps ? 1
                           : p.wide   ? (int64_t)p.W * p.R * p.C
                                      : (int64_t)(4 / p.S) * p.R;
    return (tiles + per_wg - 1) / per_wg;
}

template <int DT, int R, int S>
static hipError_t launch_rs(const GemvLaunch& a, int64_t wgs, hipStream_t stream) {
    hipLaunchKernelGGL((gemv_kernel<DT, R, S>), dim3((unsigned)wgs), dim3(kGemvThreads), 0, stream,
                       a);
    return hipGetLastError();
}

template <int DT, int MMAX, int W>
static hipError_t launch_mask(const GemvLaunch& a, int64_t wgs, hipStream_t stream) {
    hipLaunchKernelGGL((gemv_mask_kernel<DT, MMAX, W>), dim3((unsigned)wgs), dim3(64 * W), 0,
                       stream, a);
    return hipGetLastError();
}

template <int DT, int R, int MM, int W>
static hipError_t launch_ps(const GemvLaunch& a, const GemvPlan& p, int64_t wgs,
                            hipStream_t stream) {
    (void)p;  // the plan's tile groups per workgroup: kPsChunk, one
    hipLaunchKernelGGL((gemv_ps_kernel<DT, R, MM, W>), dim3((unsigned)wgs), dim3(64 * W), 0,
                       stream, a);
    return hipGetLastError();
}

template <int DT, int MM>
static hipError_t launch_psk(const GemvLaunch& a, int64_t wgs, hipStream_t stream) {
    constexpr int W = MM == 4 ? kPskWavesM4 : 4;
    hipLaunchKernelGGL((gemv_psk_kernel<DT, MM, W>), dim3((unsigned)wgs), dim3(64 * W), 0, stream,
                       a);
    return hipGetLastError();
}

template <int DT>
static hipError_t launch_dt(const GemvLaunch& a, const GemvPlan& p, int64_t wgs,
                            hipStream_t stream) {
    if (p.split_ps) {
        if (p.mmax == 1) return launch_psk<DT, 1>(a, wgs, stream);
        if (p.mmax == 4) return launch_psk<DT, 4>(a, wgs, stream);
        return hipErrorInvalidValue;
    }
    if (p.wide) {
        if (p.W == kPsWaves && p.R == kPsTiles && p.mmax == 1)
            return launch_ps<DT, kPsTiles, 1, kPsWaves>(a, p, wgs, stream);
        if (p.W == kPsWavesM4 && p.R == kPsTiles && p.mmax == 4)
            return launch_ps<DT, kPsTiles, 4, kPsWavesM4>(a, p, wgs, stream);
        if (p.W == kPsWaves && p.R == 1 && p.mmax == 4)
            return launch_ps<DT, 1, 4, kPsWaves>(a, p, wgs, stream);
        if (p.W == kMaskWaves && p.R == 2 && p.mmax == 16)
            return launch_mask<DT, 16, kMaskWaves>(a, wgs, stream);
        return hipErrorInvalidValue;
    }
    if (p.R == 1 && p.S == 2) return launch_rs<DT, 1, 2>(a, wgs, stream);
    if (p.R == 1 && p.S == 4) return launch_rs<DT, 1, 4>(a, wgs, stream);
    return hipErrorInvalidValue;
}

static hipError_t launch_tile_plan(const GemvLaunch& a, const GemvPlan& p, int64_t wgs,
                                  int dt, hipStream_t s);

hipError_t launch_gemv(const GemvLaunch& a, const GemvPlan& p, int64_t wgs, int dt,
                       hipStream_t stream) {
    if (wgs <= 0) return hipSuccess;
    if (wgs > 0x7FFFFFFF) return hipErrorInvalidValue;
    if (p.tile) return launch_tile_plan(a, p, wgs, dt, stream);
    return dt == kBF16 ? launch_dt<kBF16>(a, p, wgs, stream)
                       : launch_dt<kF16>(a, p, wgs, stream);
}

bool gemv2_supported(const void* x, const uint8_t* packed, const uint16_t* scales,
                     const void* y, int64_t M, int64_t N, int64_t K, int64_t gs, int dt, int fmt) {
    if (fmt != kFmt2Bit && fmt != kFmtRoot) return false;
    // 1-bit at M = 1 only: per-linear 8-layer stack M = 1 0.528 -> 0.456 ms, M = 4 0.548 ->
    // 0.561 ms against the B-operand kernel (same box)
    if (fmt == kFmtRoot && M != 1) return false;
    if (dt != kBF16 && dt != kF16) return false;
    if (M < 1 || M > 4 || N < 1 || K < kRound || K % kRound != 0) return false;
    if (gs != 8 && gs != 16 && gs != 32 && gs != 64) return false;
    if (((uintptr_t)x & 15u) || ((uintptr_t)packed & 15u) || ((uintptr_t)scales & 15u) ||
        ((uintptr_t)y & 1u))
        return false;
    // 32-bit buffer offsets (codes, scales, activations, with one tile of row padding)
    const int64_t rowbytes = fmt == kFmtRoot ? K / 8 : K / 4;
    if ((N + 64) * rowbytes >= (1ll << 31) || (N + 64) * (K * 2 / gs) >= (1ll << 31) ||
        M * K * 2 >= (1ll << 31))
        return false;
    return true;
}

// One linear as a launch of one inline job.
static GemvLaunch one_job(const void* x, const uint8_t* packed, const uint16_t* scales,
                          const void* bias, void* y, int M, int64_t N, int64_t K,
                          const LoraEp& lora) {
    GemvLaunch a{};
    GemvJob& j = a.inl[0];
    j.x = x; j.packed = packed; j.scales = scales; j.bias = bias; j.y = y;
    j.N = N; j.K = K; j.y_col = 0; j.y_ld = N; j.wg_begin = 0;
    j.lora_u = lora.u; j.lora_b = lora.b; j.lora_r = lora.r; j.lora_ldu = lora.ldu;
    a.njobs = 1;
    a.M = M;
    return a;
}

// `wgs` workgroups of one 16-row tile each (each job's tiles start a new workgroup)
template <int DT, int MM, int GS>
static hipError_t launch_gemv2_t(const void* x, const uint8_t* packed, const uint16_t* scales,
                                 const void* bias, void* y, int M, int64_t N, int64_t K,
                                 hipStream_t stream, const LoraEp& lora, int fmt) {
    const GemvLaunch a = one_job(x, packed, scales, bias, y, M, N, K, lora);
    const dim3 grid((unsigned)((N + 15) / 16)), block(64 * kB2Waves);
    if (fmt == kFmtRoot) {
        if constexpr (MM != 1) return hipErrorInvalidValue;  // gemv2_supported: M == 1
        else hipLaunchKernelGGL((gemv2_kernel<DT, 1, GS, kFmtRoot>), grid, block, 0, stream, a);
    } else {
        hipLaunchKernelGGL((gemv2_kernel<DT, MM, GS>), grid, block, 0, stream, a);
    }
    return hipGetLastError();
}

template <int DT, int MM>
static hipError_t launch_gemv2_gs(const void* x, const uint8_t* packed, const uint16_t* scales,
                                  const void* bias, void* y, int M, int64_t N, int64_t K,
                                  int64_t gs, hipStream_t stream, const LoraEp& lora, int fmt) {
    switch (gs) {
        case 8: return launch_gemv2_t<DT, MM, 8>(x, packed, scales, bias, y, M, N, K, stream, lora, fmt);
        case 16: return launch_gemv2_t<DT, MM, 16>(x, packed, scales, bias, y, M, N, K, stream, lora, fmt);
        case 32: return launch_gemv2_t<DT, MM, 32>(x, packed, scales, bias, y, M, N, K, stream, lora, fmt);
        default: return launch_gemv2_t<DT, MM, 64>(x, packed, scales, bias, y, M, N, K, stream, lora, fmt);
    }
}

bool gemv2m_supported(const void* x, const uint8_t* packed, const uint16_t* scales,
                      const void* y, int64_t M, int64_t N, int64_t K, int64_t gs, int dt,
                      int fmt) {
    if (fmt != kFmtTernary && fmt != kFmt2Bit && fmt != kFmtRoot) return false;
    if (fmt == kFmtTernary && gs != 16 && gs != 32 && gs != 64) return false;
    if (dt != kBF16 && dt != kF16) return false;
    if (M < 1 || M > 16 || N < 1 || K < kB2mRound || K % kB2mRound != 0) return false;
    if (gs != 8 && gs != 16 && gs != 32 && gs != 64) return false;
    if (((uintptr_t)x & 15u) || ((uintptr_t)packed & 15u) || ((uintptr_t)scales & 15u) ||
        ((uintptr_t)y & 1u))
        return false;
    const int64_t rowbytes = fmt == kFmtTernary ? K * 3 / 16 : fmt == kFmtRoot ? K / 8 : K / 4;
    if ((N + 32) * rowbytes >= (1ll << 31) ||
        (N + 32) * (K * 2 / gs) >= (1ll << 31) ||
        M * K * 2 >= (1ll << 31))
        return false;
    return true;
}

// `wgs` workgroups of R 16-row tiles each; M <= 4 stages four activation rows
template <int DT, int GS, int FMT>
static hipError_t launch_gemv2m_grid(const GemvLaunch& a, int64_t wgs, int R,
                                     hipStream_t stream) {
    if (a.M <= kB2sRows) {
        if (R == 2)
            hipLaunchKernelGGL((gemv2s_kernel<DT, GS, FMT, 2>), dim3((unsigned)wgs),
                               dim3(64 * kB2Waves), 0, stream, a);
        else
            hipLaunchKernelGGL((gemv2s_kernel<DT, GS, FMT, 1>), dim3((unsigned)wgs),
                               dim3(64 * kB2Waves), 0, stream, a);
    } else if (R == 2) {
        hipLaunchKernelGGL((gemv2m_kernel<DT, GS, FMT, 2>), dim3((unsigned)wgs),
                           dim3(64 * kB2Waves), 0, stream, a);
    } else {
        hipLaunchKernelGGL((gemv2m_kernel<DT, GS, FMT, 1>), dim3((unsigned)wgs),
                           dim3(64 * kB2Waves), 0, stream, a);
    }
    return hipGetLastError();
}

template <int DT, int GS, int FMT>
static hipError_t launch_gemv2m_t(const void* x, const uint8_t* packed, const uint16_t* scales,
                                  const void* bias, void* y, int M, int64_t N, int64_t K,
                                  hipStream_t stream, const LoraEp& lora) {
    const int64_t tiles = (N + 15) / 16;
    const GemvLaunch a = one_job(x, packed, scales, bias, y, M, N, K, lora);
    if constexpr (FMT != kFmtRoot) {
        if (M > kB2sRows && K <= kB2xMaxK) {
            // activations resident (one workgroup per CU): up to four tiles per workgroup,
            // so that the grid stays within one workgroup per CU where it can
            const int tpw = tiles > 512 ? 4 : tiles > 256 ? 2 : 1;
            const int64_t wgs = (tiles + tpw - 1) / tpw;
            if (tpw == 4)
                hipLaunchKernelGGL((gemv2x_kernel<DT, GS, FMT, 4>), dim3((unsigned)wgs),
                                   dim3(64 * kB2xWaves), 0, stream, a);
            else if (tpw == 2)
                hipLaunchKernelGGL((gemv2x_kernel<DT, GS, FMT, 2>), dim3((unsigned)wgs),
                                   dim3(64 * kB2xWaves), 0, stream, a);
            else
                hipLaunchKernelGGL((gemv2x_kernel<DT, GS, FMT, 1>), dim3((unsigned)wgs),
                                   dim3(64 * kB2xWaves), 0, stream, a);
            return hipGetLastError();
        }
    }
    if constexpr (FMT != kFmtRoot) {
        if (M > kB2sRows && K <= kB2xWaves * kB2xkRounds * kB2mRound) {
            hipLaunchKernelGGL((gemv2xk_kernel<DT, GS, FMT>), dim3((unsigned)tiles),
                               dim3(64 * kB2xWaves), 0, stream, a);
            return hipGetLastError();
        }
    }
    const int R = tiles >= kB2mTwoTilesFrom ? 2 : 1;
    return launch_gemv2m_grid<DT, GS, FMT>(a, (tiles + R - 1) / R, R, stream);
}

template <int DT, int FMT>
static hipError_t launch_gemv2m_gs(const void* x, const uint8_t* packed, const uint16_t* scales,
                                   const void* bias, void* y, int M, int64_t N, int64_t K,
                                   int64_t gs, hipStream_t stream, const LoraEp& lora) {
    switch (gs) {
        case 8: return launch_gemv2m_t<DT, 8, FMT>(x, packed, scales, bias, y, M, N, K, stream, lora);
        case 16: return launch_gemv2m_t<DT, 16, FMT>(x, packed, scales, bias, y, M, N, K, stream, lora);
        case 32: return launch_gemv2m_t<DT, 32, FMT>(x, packed, scales, bias, y, M, N, K, stream, lora);
        default: return launch_gemv2m_t<DT, 64, FMT>(x, packed, scales, bias, y, M, N, K, stream, lora);
    }
}

hipError_t launch_gemv2m(const void* x, const uint8_t* packed, const uint16_t* scales,
                         const void* bias, void* y, int64_t M, int64_t N, int64_t K, int64_t gs,
                         int dt, hipStream_t stream, int fmt, const LoraEp& lora) {
    const int m = (int)M;
    if (fmt == kFmtTernary) {  // group sizes 16, 32, 64
        if (gs == 16)
            return dt == kBF16
                       ? launch_gemv2m_t<kBF16, 16, kFmtTernary>(x, packed, scales, bias, y, m, N, K, stream, lora)
                       : launch_gemv2m_t<kF16, 16, kFmtTernary>(x, packed, scales, bias, y, m, N, K, stream, lora);
        if (gs == 64)
            return dt == kBF16
                       ? launch_gemv2m_t<kBF16, 64, kFmtTernary>(x, packed, scales, bias, y, m, N, K, stream, lora)
                       : launch_gemv2m_t<kF16, 64, kFmtTernary>(x, packed, scales, bias, y, m, N, K, stream, lora);
        return dt == kBF16
                   ? launch_gemv2m_t<kBF16, 32, kFmtTernary>(x, packed, scales, bias, y, m, N, K, stream, lora)
                   : launch_gemv2m_t<kF16, 32, kFmtTernary>(x, packed, scales, bias, y, m, N, K, stream, lora);
    }
    if (fmt == kFmtRoot)
        return dt == kBF16
                   ? launch_gemv2m_gs<kBF16, kFmtRoot>(x, packed, scales, bias, y, m, N, K, gs, stream, lora)
                   : launch_gemv2m_gs<kF16, kFmtRoot>(x, packed, scales, bias, y, m, N, K, gs, stream, lora);
    return dt == kBF16
               ? launch_gemv2m_gs<kBF16, kFmt2Bit>(x, packed, scales, bias, y, m, N, K, gs, stream, lora)
               : launch_gemv2m_gs<kF16, kFmt2Bit>(x, packed, scales, bias, y, m, N, K, gs, stream, lora);
}


// ---- staged-tile GEMV launch

// Rounds per wave (1, 2 or 4) of a staged-tile launch whose longest K has Kmax / 1024
// rounds, 0 if its stages would not fit: M == 1 up to K = 16384, M <= 4 up to K = 8192.
int gemv_tile_rounds(int64_t M, int64_t Kmax) {
    const int64_t T = Kmax / 1024;
    const int64_t U = (T + kTileWaves - 1) / kTileWaves;
    if (M < 1 || M > 4 || T < 1) return 0;
    if (U <= 1) return 1;
    if (U <= 2) return 2;
    if (U <= 4 && M == 1) return 4;
    return 0;
}

// Row tiles per workgroup of a staged-tile launch over `tiles` row tiles of K <= 4096: two
// when M == 1 and the launch has too many tiles for one-tile workgroups to be resident at
// once (their stages and table take 51 KB: three per CU), which shares the table between
// two tiles.
int gemv_tile_per_wg(int64_t M, int64_t tiles) {
    return (M == 1 && tiles >= 768) ? 2 : 1;
}

// Row tiles per wave of a staged-tile launch: two at 1 < M <= 4 with one round per wave when
// the launch has many tiles (the tiles share the activation stage, 9 KB per wave and round
// at M = 4, and the A fragment reads; the stages of a workgroup then still fit twice per CU
// with a 16-slice table).
int gemv_tile_rows_per_wave(int64_t M, int64_t tiles, int U) {
    return (M > 1 && U == 1 && tiles >= 768) ? 2 : 1;
}

bool gemv_lora_inline_ok(int U, int rt, int tpw, int64_t rank, const void* lora_a) {
    return U == 1 && rt == 1 && tpw == 1 && rank == kLoraInlineRank &&
           ((uintptr_t)lora_a & 15u) == 0;
}

bool gemv_tile_lora_inline_ok(int64_t M, int64_t N, int64_t K, int64_t rank,
                              const void* lora_a) {
    const int64_t tiles = (N + 15) / 16;
    const int U = gemv_tile_rounds(M, K);
    return gemv_lora_inline_ok(U, gemv_tile_rows_per_wave(M, tiles, U),
                               U == 1 ? gemv_tile_per_wg(M, tiles) : 1, rank, lora_a);
}

bool gemv_tile_supported(const void* x, const uint8_t* packed, const uint16_t* scales,
                         const void* y, int64_t M, int64_t N, int64_t K, int64_t gs, int dt) {
    if (dt != kBF16 && dt != kF16) return false;
    if ((gs != 16 && gs != 32 && gs != 64) || N < 1 || K < 1024 || K % 1024 != 0 ||
        gemv_tile_rounds(M, K) == 0)
        return false;
    if (((uintptr_t)x & 15u) || ((uintptr_t)packed & 15u) || ((uintptr_t)scales & 15u) ||
        ((uintptr_t)y & 1u))
        return false;
    // 32-bit buffer offsets (with one tile of row padding)
    return (N + 16) * (K * 3 / 16) < (1ll << 31) && M * K * 2 < (1ll << 31);
}

// Grouped launches below these row-tile counts take the staged-tile kernel: M == 1 and
// 1 < M <= 4 (from 1024 tiles the post-scaled kernel with one tile per wave is faster there).
GemvPlan gemv_pick_grouped(int64_t total_tiles, int64_t M, int64_t kmax, bool tile_ok) {
    const int U = tile_ok ? gemv_tile_rounds(M, kmax) : 0;
    const int64_t below = M == 1 ? 4096 : 1024;
    if (U == 0 || total_tiles >= below) return gemv_pick(total_tiles, M);
    GemvPlan p{};
    p.tile = true;
    p.U = U;
    p.rt = gemv_tile_rows_per_wave(M, total_tiles, U);
    p.tpw = (U == 1 ? gemv_tile_per_wg(M, total_tiles) : 1) * p.rt;
    p.R = p.S = p.W = p.C = 1;
    p.mmax = M == 1 ? 1 : 4;
    return p;
}

// `wgs` workgroups of TPW * RT row tiles each (each job's tiles start a new workgroup)
template <int DT, int GS, int MM, int U, int TPW, int RT, int TW = kTileWaves>
static hipError_t launch_tile_grid(const GemvLaunch& a, int64_t wgs, hipStream_t s) {
    if constexpr (U == 1 && TPW == 1 && RT == 1 && TW == kTileWaves) {
        if (a.lora_inline) {
            hipLaunchKernelGGL((gemv_tile_kernel<DT, MM, U, TPW, RT, TW, GS, true>),
                               dim3((unsigned)wgs), dim3(64 * TW * TPW), 0, s, a);
            return hipGetLastError();
        }
    }
    hipLaunchKernelGGL((gemv_tile_kernel<DT, MM, U, TPW, RT, TW, GS>), dim3((unsigned)wgs),
                       dim3(64 * TW * TPW), 0, s, a);
    return hipGetLastError();
}

// tpw: row tiles per workgroup, rt of them per wave.  Two wave sets per workgroup exist for
// U == 1 at M == 1 only (gemv_tile_per_wg), two tiles per wave for U == 1 at M > 1 only
// (gemv_tile_rows_per_wave).
template <int DT, int GS>
static hipError_t launch_tile_dt(const GemvLaunch& a, int64_t wgs, int U, int tpw, int rt,
                                 hipStream_t s) {
    if (a.M == 1) {
        if (rt != 1) return hipErrorInvalidValue;
        if (U == 1) return tpw == 2 ? launch_tile_grid<DT, GS, 1, 1, 2, 1>(a, wgs, s)
                                    : launch_tile_grid<DT, GS, 1, 1, 1, 1>(a, wgs, s);
        if (tpw != 1) return hipErrorInvalidValue;
        // a tile's rounds over 8 or 16 waves, one each (the same stage bytes per workgroup
        // as 4 waves of 2 or 4 rounds, but more waves per SIMD to run them)
        if (U == 2) return launch_tile_grid<DT, GS, 1, 1, 1, 1, 8>(a, wgs, s);
        if (U == 4) return launch_tile_grid<DT, GS, 1, 1, 1, 1, 16>(a, wgs, s);
        return hipErrorInvalidValue;
    }
    if (tpw != rt) return hipErrorInvalidValue;
    if (U == 1) return rt == 2 ? launch_tile_grid<DT, GS, 4, 1, 1, 2>(a, wgs, s)
                               : launch_tile_grid<DT, GS, 4, 1, 1, 1>(a, wgs, s);
    if (U == 2 && rt == 1) return launch_tile_grid<DT, GS, 4, 1, 1, 1, 8>(a, wgs, s);
    return hipErrorInvalidValue;
}

// Grouped launches (group size 32).
static hipError_t launch_tile_plan(const GemvLaunch& a, const GemvPlan& p, int64_t wgs,
                                   int dt, hipStream_t s) {
    return dt == kBF16 ? launch_tile_dt<kBF16, 32>(a, wgs, p.U, p.tpw, p.rt, s)
                       : launch_tile_dt<kF16, 32>(a, wgs, p.U, p.tpw, p.rt, s);
}
template <int GS>
static hipError_t launch_gemv_tile_gs(const GemvLaunch& a, int64_t wgs, int U, int tpw, int rt,
                                      int dt, hipStream_t s) {
    return dt == kBF16 ? launch_tile_dt<kBF16, GS>(a, wgs, U, tpw, rt, s)
                       : launch_tile_dt<kF16, GS>(a, wgs, U, tpw, rt, s);
}

// One job of `tiles` row tiles (per-linear launch) at group size gs (16, 32 or 64).
hipError_t launch_gemv_tile(const GemvLaunch& a, int64_t tiles, int64_t Kmax, int dt,
                            hipStream_t s, int64_t gs) {
    if (tiles <= 0) return hipSuccess;
    const int U = gemv_tile_rounds(a.M, Kmax);
    if (tiles > 0x7FFFFFFF || U == 0) return hipErrorInvalidValue;
    const int rt = gemv_tile_rows_per_wave(a.M, tiles, U);
    const int tpw = (U == 1 ? gemv_tile_per_wg(a.M, tiles) : 1) * rt;
    const int64_t wgs = (tiles + tpw - 1) / tpw;
    if (gs == 16) return launch_gemv_tile_gs<16>(a, wgs, U, tpw, rt, dt, s);
    if (gs == 64) return launch_gemv_tile_gs<64>(a, wgs, U, tpw, rt, dt, s);
    return launch_gemv_tile_gs<32>(a, wgs, U, tpw, rt, dt, s);
}

hipError_t launch_gemv2(const void* x, const uint8_t* packed, const uint16_t* scales,
                        const void* bias, void* y, int64_t M, int64_t N, int64_t K, int64_t gs,
                        int dt, hipStream_t stream, const LoraEp& lora, int fmt) {
    const int m = (int)M;
    if (dt == kBF16)
        return M == 1 ? launch_gemv2_gs<kBF16, 1>(x, packed, scales, bias, y, m, N, K, gs, stream, lora, fmt)
                      : launch_gemv2_gs<kBF16, 4>(x, packed, scales, bias, y, m, N, K, gs, stream, lora, fmt);
    return M == 1 ? launch_gemv2_gs<kF16, 1>(x, packed, scales, bias, y, m, N, K, gs, stream, lora, fmt)
                  : launch_gemv2_gs<kF16, 4>(x, packed, scales, bias, y, m, N, K, gs, stream, lora, fmt);
}

// ---- streaming 2-bit and 1-bit GEMV for grouped launches
//
// The per-linear 2-bit kernels above give each workgroup one or two 16-row tiles and split
// K over its waves, so every workgroup stages the activations of all of K for 16-32 rows:
// in a grouped launch over a whole stack that re-reads x from L2 more often than the
// weights themselves (at M = 4, 32 KB of x against 20 KB of weights per K = 4096 tile).
// Here the W waves of a workgroup own R row tiles each over all of K and share one
// activation stage per round (W * R * 16 rows per x round), with one barrier per round.
// Each lane loads its codes and scales of the next round into registers while the current
// round computes (the per-linear kernels' load pattern: 64 contiguous bytes of 16 rows per
// instruction).  MM <= 4: post-scaled 1024-k rounds (B2Round over the byte table, R tiles
// sharing each A fragment; the nibble table's four reads and address computations per 8
// weights made the kernel VALU- and LDS-issue-bound: 17.2 VALU and 5.0 LDS instructions per
// MFMA against 10.5 and 2.5, M = 4 stack 0.725 -> 0.605 ms, same box); MM = 16: the
// B-operand 256-k rounds (B2mRound, R tiles sharing each A fragment).  1-bit codes take the
// same rounds with 8-byte code pieces per lane and the 1-bit tables.
// G (B-operand form): rounds per load group.  A 256-k round takes 64 bytes of a 2-bit row and
// 32 bytes of a 1-bit row, so 2 or 4 consecutive rounds share each 128-byte line; fetched one
// round at a time, a line's later parts were requested a round after its first, often after
// L2 had evicted it (traffic 1.8x / 2.7x the algorithmic bytes at M = 16).  A group's rounds
// are requested back to back and computed in turn (every K % (256 G) == 0): 32-layer stack
// at M = 16, 2-bit (G = 2) 0.66 -> 0.62 ms, 1-bit (G = 4) 0.568 -> 0.547 ms (one tile per
// wave instead: 0.66 and 0.62 ms).
template <int DT, int GS, int MM, int R, int W, int FMT = kFmt2Bit, int G = 1>
__global__ __launch_bounds__(64 * W) void gemv2g_kernel(GemvLaunch args) {
    constexpr bool kPost = MM <= 4;
    static_assert(G == 1 || !kPost, "load groups in the B-operand form only");
    // 1-bit Root E8 (FMT kFmtRoot): post-scaled with its code -> coordinates table, or the
    // B-operand form with its code -> selector table
    static_assert(FMT == kFmt2Bit || FMT == kFmtRoot, "2-bit or 1-bit codes");
    static_assert(MM == 1 || MM == 4 || MM == 16, "activation rows 1, 4 or 16");
    constexpr int kXBytes = kPost ? MM * (int)kXRow : kB2mXBytes;  // one round's stage
    // table copies (lane l reads copy l % BC): 16 of the 2-bit byte tables, whose 8-byte
    // entries hold four weights (post-scaled) or two selector words (B operand; 32 copies,
    // conflict-free, measured 2% slower at M = 1); one of the 4 KB 1-bit tables, whose
    // 16-byte entries hold a code's coordinates (post-scaled) or selector words (B operand):
    // more copies cost more than their bank conflicts (32-layer stack, coordinates copied
    // from the compile-time table: 0.408 ms at M = 1 with one copy, 0.417 / 0.422 / 0.448 with
    // 2 / 4 / 8; selectors 0.569 against 0.585 ms with 8)
    constexpr int BC = FMT == kFmtRoot ? 1 : 16;
    __shared__ uint4 lut_storage[FMT == kFmtRoot ? kSel1Entries * BC : kB2ByteLutU4<16>];
    // two activation stages, separate LDS objects; the post-scaled ones end in a zero block
    // (the A fragments of lanes outside their lane group)
    __shared__ __attribute__((aligned(128))) char xs0[G * kXBytes + (kPost ? kB2ZeroBytes : 0)];
    __shared__ __attribute__((aligned(128))) char xs1[G * kXBytes + (kPost ? kB2ZeroBytes : 0)];

    if constexpr (kPost) {
        if constexpr (FMT == kFmtRoot) fill_v1<DT, BC, 64 * W>(lut_storage);
        else fill_b2blut<DT, 64 * W, BC>(lut_storage);
        for (int i = (int)threadIdx.x; i < kB2ZeroBytes / 16; i += 64 * W) {
            reinterpret_cast<uint4*>(xs0 + kXBytes)[i] = make_uint4(0u, 0u, 0u, 0u);
            reinterpret_cast<uint4*>(xs1 + kXBytes)[i] = make_uint4(0u, 0u, 0u, 0u);
        }
    } else {
        if constexpr (FMT == kFmtRoot) fill_sel1<64 * W, BC>(lut_storage);
        else fill_b2bsel<64 * W, BC>(lut_storage);
    }

    int64_t wg = blockIdx.x;
    const GemvJob job = gemv_job_of(args, wg);
    const void* const x = job.x ? job.x : args.x;
    void* const y = job.y ? job.y : args.y;
    const int M = args.M;
    const int64_t N = job.N, K = job.K;
    const LoraEp lora{job.lora_u, job.lora_b, job.lora_r,
                      job.lora_ldu ? job.lora_ldu : job.lora_r, job.N};

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int g = lane >> 4, i16 = lane & 15;
    const int64_t tile0 = (wg * W + wave) * R;
    const uint32_t rowbytes = (uint32_t)(FMT == kFmtRoot ? K / 8 : K / 4);
    const uint32_t srowbytes = (uint32_t)(K * 2 / GS);
    constexpr uint32_t kLaneBytes = FMT == kFmtRoot ? 8u : 16u;  // a lane's codes per round
    const __amdgpu_buffer_rsrc_t pr = __builtin_amdgcn_make_buffer_rsrc(
        (void*)job.packed, (short)0, (int)(N * rowbytes), kRsrcWord3);
    const __amdgpu_buffer_rsrc_t sr = __builtin_amdgcn_make_buffer_rsrc(
        (void*)job.scales, (short)0, (int)(N * srowbytes), kRsrcWord3);
    const __amdgpu_buffer_rsrc_t xr = __builtin_amdgcn_make_buffer_rsrc(
        (void*)x, (short)0, (int)(M * K * 2), kRsrcWord3);
    // rows past N read zeros (buffer bound) and are never stored
    uint32_t vo_code[R], vo_scale[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const uint32_t row = (uint32_t)((tile0 + r) * 16 + i16);
        vo_code[r] = row * rowbytes + kLaneBytes * g;
        vo_scale[r] = row * srowbytes + (128u / GS) * g;
    }
    const uint32_t slot = FMT == kFmtRoot ? (uint32_t)(lane & (BC - 1)) * 16u : b2_slot<BC>(lane);
    const int T = (int)(K / (kPost ? kRound : kB2mRound));

    // this lane's activation reads: post-scaled A row i16 = 4 g' + m is live in lane group g'
    // only (others read the zero block); B-operand: the swizzled 16-row stage
    const int am = i16 & 3;
    const bool a_live = (i16 >> 2) == g && am < M;
    const int aoff = a_live ? am * (int)kXRow + 128 * g : kXBytes;
    const uint32_t gu = (uint32_t)g, iu = (uint32_t)i16;
    const uint32_t xo = 512u * iu + 16u * ((8u * gu & 16u) | ((8u * gu & 8u) ^ (iu & 8u)) | (iu & 7u));
    uint32_t xo_ld[8];
    if constexpr (!kPost) {
#pragma unroll
        for (int q = 0; q < 8; ++q) xo_ld[q] = b2m_x_offset(q, lane, M, K);
    }

    // the workgroup's share of one round's activation loads: post-scaled 2 MM 1-KB loads
    // (rows m >= M re-read row M - 1 into rows no lane reads), B-operand eight
    auto stage = [&](char* xs, int u) {
        if constexpr (kPost) {
            for (int q = wave; q < 2 * MM; q += W) {
                const int m = q >> 1, half = q & 1;
                const int msrc = m < M ? m : M - 1;
                __builtin_amdgcn_raw_ptr_buffer_load_lds(
                    xr, lds_ptr(xs + m * kXRow + half * 1024), 16,
                    (uint32_t)(msrc * K * 2 + half * 1024 + lane * 16),
                    uniform_offset((int64_t)u * kRound * 2), 0, 0);
            }
        } else {
            for (int q = wave; q < 8; q += W)
                __builtin_amdgcn_raw_ptr_buffer_load_lds(xr, lds_ptr(xs + 1024 * q), 16, xo_ld[q],
                                                         uniform_offset((int64_t)u * kB2mRound * 2),
                                                         0, 0);
        }
    };
    using Piece = std::conditional_t<kPost, uint4[4], uint4>;
    Piece cp0[G][R], sp0[G][R], cp1[G][R], sp1[G][R];
    auto load = [&](Piece (&cp)[R], Piece (&sp)[R], int u) {
#pragma unroll
        for (int r = 0; r < R; ++r) {
            if constexpr (kPost && FMT == kFmtRoot)
                b1_load<GS>(cp[r], sp[r], pr, sr, vo_code[r], vo_scale[r], u);
            else if constexpr (kPost)
                b2_load<GS>(cp[r], sp[r], pr, sr, vo_code[r], vo_scale[r], u);
            else b2m_load<GS, FMT>(cp[r], sp[r], pr, sr, vo_code[r], vo_scale[r], u);
        }
    };
    float accp[R][kPost ? MM : 1];
    f32x4 accm[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
        accm[r] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int q = 0; q < (kPost ? MM : 1); ++q) accp[r][q] = 0.f;
    }
    const char* lut = reinterpret_cast<const char*>(lut_storage);
    auto compute = [&](const Piece (&cp)[R], const Piece (&sp)[R], const char* xs) {
        if constexpr (kPost) {
            B2Round<DT, MM, GS, R, BC, FMT>::run(cp, sp, lut, slot, xs + aoff, accp);
        } else {
            B2mRound<DT, GS, FMT, R, BC>::run(cp, sp, lut, slot, xs, xo, accm);
        }
    };

    // load group v: rounds G v .. G v + G - 1 (codes and scales, then their activations)
    auto fetch = [&](Piece (&cp)[G][R], Piece (&sp)[G][R], char* xs, int v) {
#pragma unroll
        for (int j = 0; j < G; ++j) load(cp[j], sp[j], G * v + j);
#pragma unroll
        for (int j = 0; j < G; ++j) stage(xs + j * kXBytes, G * v + j);
    };
    auto compute_group = [&](const Piece (&cp)[G][R], const Piece (&sp)[G][R], const char* xs) {
#pragma unroll
        for (int j = 0; j < G; ++j) compute(cp[j], sp[j], xs + j * kXBytes);
    };
    const int TG = T / G;

    fetch(cp0, sp0, xs0, 0);
    vm_wait_all();
    __syncthreads();  // table, zero blocks, load group 0 ready
    // load groups in pairs, so that each register set and stage is a compile-time choice;
    // group v fetches group v + 1 while it computes, then the workgroup waits for it
    for (int v = 0; v < TG; v += 2) {
        if (v + 1 < TG) fetch(cp1, sp1, xs1, v + 1);
        compute_group(cp0, sp0, xs0);
        vm_wait_all();
        __syncthreads();
        if (v + 1 >= TG) break;
        if (v + 2 < TG) fetch(cp0, sp0, xs0, v + 2);
        compute_group(cp1, sp1, xs1);
        vm_wait_all();
        __syncthreads();
    }

#pragma unroll
    for (int r = 0; r < R; ++r) {
        const int64_t row = (tile0 + r) * 16 + i16;
        if constexpr (kPost) {
            // the four lane groups of each row; lane group q keeps activation row q
            float out = 0.f;
#pragma unroll
            for (int q = 0; q < MM; ++q) {
                float v = accp[r][q];
                v += __shfl_xor(v, 16);
                v += __shfl_xor(v, 32);
                if (q == g) out = v;
            }
            if (row < N && g < M) {
                const float bv = job.bias ? load_as_f32<DT>(job.bias, row) : 0.f;
                store_from_f32<DT>(y, (int64_t)g * job.y_ld + job.y_col + row,
                                   out + bv + lora_term<DT>(lora, g, row));
            }
        } else if (row < N) {
            // lane (g, n) holds rows m = 4g + q of column n
            const float bv = job.bias ? load_as_f32<DT>(job.bias, row) : 0.f;
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const int m = 4 * g + q;
                if (m < M)
                    store_from_f32<DT>(y, (int64_t)m * job.y_ld + job.y_col + row,
                                       accm[r][q] + bv + lora_term<DT>(lora, m, row));
            }
        }
    }
}

// ---- grouped 2-bit / 1-bit decode GEMV: many linears of one group size in one launch
// Streaming kernel geometry of a grouped launch: waves per workgroup and row tiles per wave;
// M <= 4 needs every K a multiple of 1024 (post-scaled rounds), otherwise the 16-row
// B-operand rounds take it.
// Measured (32-layer stack, same box): 2-bit post-scaled 4 waves x 2 tiles (8 x 1 equal,
// 8 x 2 0.536 -> 0.646 ms at M = 1); B operand 8 waves x 2 tiles (0.674 -> 0.659 ms at
// M = 16).  1-bit post-scaled 4 waves x 2 tiles: 0.478 ms at M = 1 against 0.50 with 3 or 4
// tiles and 0.59-0.61 with 8 waves.
constexpr int kB2gWaves = 4;
constexpr int kB2gWavesB = 8;
constexpr int kB2gTiles = 2;
constexpr int kB1gTiles = 2;  // 1-bit post-scaled
constexpr int kB1gWaves = 4;
// B-operand form where every K % 1024 == 0: rounds per load group (2-bit, 1-bit)
constexpr int kB2gGroupB2 = 2;
constexpr int kB2gGroupB1 = 4;
Gemv2Plan gemv2_pick_grouped(int64_t total_tiles, int64_t M, bool k1024, int fmt) {
    (void)total_tiles;
    Gemv2Plan p{};
    p.post = M <= 4 && k1024;
    p.grouped_rounds = !p.post && k1024;
    // row tiles per workgroup
    p.R = !p.post ? kB2gWavesB * kB2gTiles
                  : fmt == kFmtRoot ? kB1gWaves * kB1gTiles : kB2gWaves * kB2gTiles;
    return p;
}
int64_t gemv2_wgs_for(int64_t N, const Gemv2Plan& p) { return ((N + 15) / 16 + p.R - 1) / p.R; }

template <int DT, int GS>
static hipError_t launch_gemv2_grouped_t(const GemvLaunch& a, const Gemv2Plan& p, int64_t wgs,
                                         int fmt, hipStream_t s) {
    if (fmt == kFmtRoot) {
        if (p.post && a.M == 1)
            hipLaunchKernelGGL((gemv2g_kernel<DT, GS, 1, kB1gTiles, kB1gWaves, kFmtRoot>),
                               dim3((unsigned)wgs), dim3(64 * kB1gWaves), 0, s, a);
        else if (p.post)
            hipLaunchKernelGGL((gemv2g_kernel<DT, GS, 4, kB1gTiles, kB1gWaves, kFmtRoot>),
                               dim3((unsigned)wgs), dim3(64 * kB1gWaves), 0, s, a);
        else if (p.grouped_rounds)
            hipLaunchKernelGGL(
                (gemv2g_kernel<DT, GS, 16, kB2gTiles, kB2gWavesB, kFmtRoot, kB2gGroupB1>),
                dim3((unsigned)wgs), dim3(64 * kB2gWavesB), 0, s, a);
        else
            hipLaunchKernelGGL((gemv2g_kernel<DT, GS, 16, kB2gTiles, kB2gWavesB, kFmtRoot>),
                               dim3((unsigned)wgs), dim3(64 * kB2gWavesB), 0, s, a);
    } else if (p.post) {
        if (a.M == 1)
            hipLaunchKernelGGL((gemv2g_kernel<DT, GS, 1, kB2gTiles, kB2gWaves>), dim3((unsigned)wgs),
                               dim3(64 * kB2gWaves), 0, s, a);
        else
            hipLaunchKernelGGL((gemv2g_kernel<DT, GS, 4, kB2gTiles, kB2gWaves>), dim3((unsigned)wgs),
                               dim3(64 * kB2gWaves), 0, s, a);
    } else if (p.grouped_rounds) {
        hipLaunchKernelGGL(
            (gemv2g_kernel<DT, GS, 16, kB2gTiles, kB2gWavesB, kFmt2Bit, kB2gGroupB2>),
            dim3((unsigned)wgs), dim3(64 * kB2gWavesB), 0, s, a);
    } else {
        hipLaunchKernelGGL((gemv2g_kernel<DT, GS, 16, kB2gTiles, kB2gWavesB>), dim3((unsigned)wgs),
                           dim3(64 * kB2gWavesB), 0, s, a);
    }
    return hipGetLastError();
}
template <int DT>
static hipError_t launch_gemv2_grouped_dt(const GemvLaunch& a, const Gemv2Plan& p, int64_t wgs,
                                          int64_t gs, int fmt, hipStream_t s) {
    switch (gs) {
        case 8: return launch_gemv2_grouped_t<DT, 8>(a, p, wgs, fmt, s);
        case 16: return launch_gemv2_grouped_t<DT, 16>(a, p, wgs, fmt, s);
        case 32: return launch_gemv2_grouped_t<DT, 32>(a, p, wgs, fmt, s);
        case 64: return launch_gemv2_grouped_t<DT, 64>(a, p, wgs, fmt, s);
        default: return hipErrorInvalidValue;
    }
}
hipError_t launch_gemv2_grouped(const GemvLaunch& a, const Gemv2Plan& p, int64_t wgs,
                                int64_t gs, int dt, int fmt, hipStream_t s) {
    if (wgs <= 0) return hipSuccess;
    if (fmt != kFmt2Bit && fmt != kFmtRoot) return hipErrorInvalidValue;
    return dt == kBF16 ? launch_gemv2_grouped_dt<kBF16>(a, p, wgs, gs, fmt, s)
                       : launch_gemv2_grouped_dt<kF16>(a, p, wgs, gs, fmt, s);
}

}  // namespace ojx
