// e8t_gemm_mfma.hip -- prefill fused ternary-E8 GEMM for gfx950 (batch M > 16).
//
// Y[M,N] = X[M,K] . Wq[N,K]^T (+ bias), Wq[n,k] = coord(code) * scale(n, k/32) in the
// activation dtype (bf16: coord * bf16_rne(s16), lattice.py:414-418), fp32 accumulation.
// Replaces the reference's TileLang ternary GEMM (tilelang_kernels.py:277-363, 64x64x64
// tiles, LUT gathered from global memory) and its unpack + dense-GEMM fallback
// (lattice.py:610-640): the weight tile is decoded once per workgroup into LDS and fed
// to bf16 MFMA, so no dense weight ever reaches HBM.
//
// Tiling.  256x256 output tile per workgroup, K step 64, 8 waves in a 2x4 grid, each
// wave 128x64 = 8x4 v_mfma_f32_16x16x32 tiles (128 fp32 accumulators per lane), so two
// waves fit on each SIMD and cover each other's LDS and barrier waits.
//   * X tile (256 x 64 bf16 = 32 KB) arrives by buffer->LDS loads, one K step ahead.
//   * W tile: each pair of threads owns one of the 256 weight rows of the tile, loads
//     its 8 codes (12 bytes) and 2 scales two K steps ahead, and each thread expands 4
//     of them through the bank-sliced LDS table (e8t_lut.h) one step ahead, writing 64
//     bytes of bf16 weights.
//   * Both tiles are double buffered; rows are stored as 8 pieces of 16 bytes with piece
//     p of row r at position p ^ ((r >> 1) & 7), which makes the 16-lane fragment reads
//     and the row writes bank-conflict free.  One barrier per K step.
// Workgroup order: consecutive workgroup ids land on different XCDs (round robin); the
// tile index is remapped so that each XCD walks a contiguous, M-grouped range of tiles
// and its L2 serves the X rows and weight columns that its concurrent workgroups share.

#include <type_traits>

#include "e8t_device.h"
#include "e8t_internal.h"
#include "e8t_lut.h"
#include "e8t_root.h"

namespace ojx {

constexpr int kBK = 64;
constexpr int kXcds = 8;
constexpr int kGroupM = 8;  // M tiles per group of the tile order
constexpr int64_t kGroup4FromTn = 32;  // column tiles from which groups hold 4

// Tile configuration: BM x BN output tile per workgroup, WAVES_M x WAVES_N waves of
// (BM / WAVES_M) x (BN / WAVES_N) each.  Two threads decode each weight row of the tile.
template <int BM_, int BN_, int WAVES_M_, int WAVES_N_>
struct GemmCfg {
    static constexpr int BM = BM_, BN = BN_;
    static constexpr int WAVES_M = WAVES_M_, WAVES_N = WAVES_N_, WAVES = WAVES_M_ * WAVES_N_;
    static constexpr int THREADS = 64 * WAVES;
    static constexpr int WM = BM / WAVES_M, WN = BN / WAVES_N;  // wave tile
    static constexpr int TM = WM / 16, TN = WN / 16;            // MFMA tiles per wave
    static constexpr int XTILE = BM * kBK * 2, WTILE = BN * kBK * 2;  // bytes per operand tile
    static constexpr int XLOADS = BM / (8 * WAVES);             // 1-KB X loads per wave
    static_assert(THREADS == 2 * BN, "two threads per weight row");
    static_assert(XLOADS * 8 * WAVES == BM, "X tile rows split evenly over the waves");
    static_assert(TM >= 4, "decode writes are spread over the last four MFMA rows");
};
using CfgLarge = GemmCfg<256, 256, 2, 4>;  // 8 waves of 128 x 64: large grids
using CfgSmall = GemmCfg<128, 128, 2, 2>;  // 4 waves of 64 x 64: grids under one wave

__device__ __forceinline__ uint32_t swz(uint32_t row, uint32_t piece) {
    return row * 128u + 16u * (piece ^ ((row >> 1) & 7u));
}

// X tile rows [m0, m0+BM) x k [k0, k0+64) -> LDS tile (swizzled); each wave issues
// `loads` 1-KB loads (8 rows each).  Rows >= M read past the buffer's end: zeros.
__device__ __forceinline__ void load_x_tile(char* tile, __amdgpu_buffer_rsrc_t x, int64_t m0,
                                            int64_t k0, int64_t K, int wave, int lane,
                                            int loads) {
    const uint32_t r_in = (uint32_t)lane >> 3, q = (uint32_t)lane & 7u;
#pragma unroll
    for (int i = 0; i < loads; ++i) {
        const uint32_t row0 = 8u * (uint32_t)(loads * wave + i);
        const uint32_t row = row0 + r_in;
        const uint32_t p = q ^ ((row >> 1) & 7u);
        const uint32_t voff = (uint32_t)((m0 + row) * K * 2 + 16u * p);
        __builtin_amdgcn_raw_ptr_buffer_load_lds(
            x, (__attribute__((address_space(3))) void*)(tile + row0 * 128), 16, voff,
            uniform_offset(k0 * 2), 0, 0);
    }
}

struct RowCodes {
    uint32_t d[3];  // 8 codes of this thread's weight row for one K step
    uint32_t s[2];  // the step's group scales (fp16 bits): 4 at GS 16, 2 at GS 32, 1 at GS 64
};

// Codes and scales of K step k0 of this thread's row (group size GS: 64 / GS scales, or the
// one scale a GS = 64 group shares between two steps).
template <int GS>
__device__ __forceinline__ void load_codes_row(RowCodes& rc, __amdgpu_buffer_rsrc_t packed,
                                               __amdgpu_buffer_rsrc_t scales, uint32_t vo_code,
                                               uint32_t vo_scale, int64_t k0) {
    static_assert(GS == 16 || GS == 32 || GS == 64, "ternary group size 16, 32 or 64");
    const u32x3 v =
        __builtin_amdgcn_raw_buffer_load_b96(packed, vo_code, uniform_offset(k0 * 3 / 16), 0);
    rc.d[0] = v.x;
    rc.d[1] = v.y;
    rc.d[2] = v.z;
    const int so = uniform_offset(k0 * 2 / GS);
    if constexpr (GS == 16) {
        const u32x2 sv = __builtin_amdgcn_raw_buffer_load_b64(scales, vo_scale, so, 0);
        rc.s[0] = sv[0];
        rc.s[1] = sv[1];
    } else if constexpr (GS == 32) {
        rc.s[0] = __builtin_amdgcn_raw_buffer_load_b32(scales, vo_scale, so, 0);
    } else {
        rc.s[0] = __builtin_amdgcn_raw_buffer_load_b16(scales, vo_scale, so, 0);
    }
}

template <int DT, int TN>
__device__ __forceinline__ void mma_row(const uint4& a, const uint4 (&b)[TN], f32x4 (&acc)[TN]) {
#pragma unroll
    for (int j = 0; j < TN; ++j) acc[j] = mfma16<DT>(a, b[j], acc[j]);
}

// Fragment addresses.  Rows of a wave's A (B) fragments are arow0 + 16i + i16 (brow0 +
// 16j + i16) with arow0, brow0 multiples of 64, so the swizzle term (row >> 1) & 7 is
// (i16 >> 1) & 7 for every fragment of a lane: each fragment is a per-lane base plus the
// compile-time offset 2048*i (one ds_read_b128 with an immediate offset).
struct FragLane {
    uint32_t a[2], b[2];  // byte offsets within a tile for K sub-step 0 / 1
};

__device__ __forceinline__ FragLane frag_lane(uint32_t arow0, uint32_t brow0, int g, int i16) {
    const uint32_t c = ((uint32_t)i16 >> 1) & 7u;
    FragLane f;
    f.a[0] = (arow0 + i16) * 128u + 16u * ((uint32_t)g ^ c);
    f.a[1] = (arow0 + i16) * 128u + 16u * ((4u + g) ^ c);
    f.b[0] = (brow0 + i16) * 128u + 16u * ((uint32_t)g ^ c);
    f.b[1] = (brow0 + i16) * 128u + 16u * ((4u + g) ^ c);
    return f;
}

template <int TM, int TN>
__device__ __forceinline__ void load_frags(const char* xt, const char* wt, const FragLane& f,
                                           int sub, uint4 (&a)[TM], uint4 (&b)[TN]) {
    const char* pa = xt + f.a[sub];
    const char* pb = wt + f.b[sub];
#pragma unroll
    for (int i = 0; i < TM; ++i) a[i] = *reinterpret_cast<const uint4*>(pa + 2048 * i);
#pragma unroll
    for (int j = 0; j < TN; ++j) b[j] = *reinterpret_cast<const uint4*>(pb + 2048 * j);
}

// Table reads of code j (0..7) of this thread's row (two 8-byte masks).
template <int J>
__device__ __forceinline__ void lut_read(const RowCodes& rc, const char* lut, uint32_t slot,
                                         uint2& ml, uint2& mh) {
    const uint32_t z = code_z<J>(rc.d, slot);
    const uint32_t h = __umulhi(z, kHiMagic);
    ml = *reinterpret_cast<const uint2*>(lut + lo_addr_of(h, z));
    mh = *reinterpret_cast<const uint2*>(lut + (h * kLutStride + slot));
}

// Table reads for codes 4*half .. 4*half+3 of this thread's row.
__device__ __forceinline__ void lut_reads_half(const RowCodes& rc, const char* lut,
                                               uint32_t slot, int half, uint2 (&ml)[4],
                                               uint2 (&mh)[4]) {
    if (half == 0) {
        lut_read<0>(rc, lut, slot, ml[0], mh[0]);
        lut_read<1>(rc, lut, slot, ml[1], mh[1]);
        lut_read<2>(rc, lut, slot, ml[2], mh[2]);
        lut_read<3>(rc, lut, slot, ml[3], mh[3]);
    } else {
        lut_read<4>(rc, lut, slot, ml[0], mh[0]);
        lut_read<5>(rc, lut, slot, ml[1], mh[1]);
        lut_read<6>(rc, lut, slot, ml[2], mh[2]);
        lut_read<7>(rc, lut, slot, ml[3], mh[3]);
    }
}

// ---- weight-row decoders: each thread owns half of one weight row of the tile (32 k of a
// 64-k step) and produces its four 16-byte pieces of activation-dtype weights.
//   load(k0)  issue the loads of the codes/scales of K step k0 (two steps ahead);
//   prep()    table reads and scale words for the codes loaded earlier (one step ahead);
//   piece(p)  the p-th 16-byte piece (8 weights) from what prep() read.

// Ternary E8: 8 codes (12 bytes) of the whole row per step; the thread expands 4 of them
// (32 k: two scale groups at GS 16, one at GS 32, half of one at GS 64).
template <int DT, int GS>
struct TernaryRowDecoder {
    static constexpr int kLoads = 2;  // loads issued by load()
    RowCodes rc;
    uint2 ml[4], mh[4];
    uint32_t sw[2];  // scale words of pieces 0-1 and 2-3
    const char* lut;
    uint32_t slot, vo_code, vo_scale;
    __amdgpu_buffer_rsrc_t pr, sr;
    int half;
    __device__ __forceinline__ void load(int64_t k0) {
        load_codes_row<GS>(rc, pr, sr, vo_code, vo_scale, k0);
    }
    __device__ __forceinline__ void prep() {
        lut_reads_half(rc, lut, slot, half, ml, mh);
        if constexpr (GS == 16) {
            scale_words<DT>(half ? rc.s[1] : rc.s[0], sw[0], sw[1]);
        } else {
            uint32_t w0, w1;
            scale_words<DT>(rc.s[0], w0, w1);
            sw[0] = sw[1] = (GS == 32 && half) ? w1 : w0;
        }
    }
    __device__ __forceinline__ uint4 piece(int p) const {
        const uint32_t s = sw[p >> 1];
        return make_uint4(ml[p].x & s, ml[p].y & s, mh[p].x & s, mh[p].y & s);
    }
    __device__ __forceinline__ void store(int p, char* tile, uint32_t wrow, int hf) const {
        *reinterpret_cast<uint4*>(tile + swz(wrow, 4u * hf + p)) = piece(p);
    }
};

// 2-bit E8 (E8LatticePacker, lattice.py:252-279): code c in {0..3} is the weight
// (c - 1.5) * s, rounded once to the activation dtype (s = scales.to(dtype)).  Per scale
// group the four possible weights are -B, -A, +A, +B with A = rnd(0.5 s), B = rnd(1.5 s)
// (the products are exact in fp32; -rnd(x) = rnd(-x)); they form the 8-byte table
// {S0 = A | B << 16, S1 = -B | -A << 16} whose byte pair 2c, 2c + 1 is the weight of code
// c.  One v_perm_b32 then yields two weights from a selector word; the selector words of a
// code byte (4 codes) come from a 256-entry LDS table (2 KB, `kSel2Entries`).
constexpr int kSel2Entries = 256;

__device__ __forceinline__ void fill_sel2(uint2* tab, int nthreads) {
    for (int e = (int)threadIdx.x; e < kSel2Entries; e += nthreads) {
        uint32_t w[2];
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const uint32_t c0 = ((uint32_t)e >> (4 * h)) & 3u, c1 = ((uint32_t)e >> (4 * h + 2)) & 3u;
            w[h] = (2u * c0) | ((2u * c0 + 1u) << 8) | ((2u * c1) << 16) | ((2u * c1 + 1u) << 24);
        }
        tab[e] = make_uint2(w[0], w[1]);
    }
}

template <int DT, int GS>
struct Bit2RowDecoder {
    static_assert(GS == 8 || GS == 16 || GS == 32 || GS == 64, "2-bit group size 8..64");
    static constexpr int kLoads = 2;
    uint2 c;          // the half-row's 32 codes (8 bytes)
    uint2 sc;         // its scales: GS 8: four, GS 16: two, GS 32/64: one (fp16 bits)
    uint2 sel[4][2];  // selector words of pieces 0..3
    uint2 val[4];     // value words of pieces 0..3
    const char* tab;
    uint32_t vo_code, vo_scale;  // this thread's half-row (codes) and scale bytes
    __amdgpu_buffer_rsrc_t pr, sr;
    __device__ __forceinline__ void load(int64_t k0) {
        const auto v = __builtin_amdgcn_raw_buffer_load_b64(pr, vo_code, uniform_offset(k0 / 4), 0);
        c = make_uint2(v[0], v[1]);
        const int so = uniform_offset(k0 * 2 / GS);
        if constexpr (GS == 8) {
            const auto u = __builtin_amdgcn_raw_buffer_load_b64(sr, vo_scale, so, 0);
            sc = make_uint2(u[0], u[1]);
        } else if constexpr (GS == 16) {
            sc = make_uint2(__builtin_amdgcn_raw_buffer_load_b32(sr, vo_scale, so, 0), 0u);
        } else {
            sc = make_uint2(__builtin_amdgcn_raw_buffer_load_b16(sr, vo_scale, so, 0), 0u);
        }
    }
    __device__ __forceinline__ void prep() {
#pragma unroll
        for (int p = 0; p < 4; ++p) {
            const uint32_t w = p < 2 ? c.x : c.y;
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const uint32_t byte = (w >> (16 * (p & 1) + 8 * h)) & 0xFFu;
                sel[p][h] = *reinterpret_cast<const uint2*>(tab + 8u * byte);
            }
        }
        if constexpr (GS == 8) {
            val[0] = values2<DT>(sc.x);
            val[1] = values2<DT>(sc.x >> 16);
            val[2] = values2<DT>(sc.y);
            val[3] = values2<DT>(sc.y >> 16);
        } else if constexpr (GS == 16) {
            val[0] = val[1] = values2<DT>(sc.x);
            val[2] = val[3] = values2<DT>(sc.x >> 16);
        } else {
            val[0] = val[1] = val[2] = val[3] = values2<DT>(sc.x);
        }
    }
    __device__ __forceinline__ uint4 piece(int p) const {
        const uint32_t s0 = val[p].x, s1 = val[p].y;
        return make_uint4(__builtin_amdgcn_perm(s0, s1, sel[p][0].x),
                          __builtin_amdgcn_perm(s0, s1, sel[p][0].y),
                          __builtin_amdgcn_perm(s0, s1, sel[p][1].x),
                          __builtin_amdgcn_perm(s0, s1, sel[p][1].y));
    }
    __device__ __forceinline__ void store(int p, char* tile, uint32_t wrow, int hf) const {
        *reinterpret_cast<uint4*>(tile + swz(wrow, 4u * hf + p)) = piece(p);
    }
};

// 1-bit Root E8 (RootE8LatticePacker, lattice.py:426-533): one code byte per 8 weights,
// coordinates 0, +-1, +-2 times the group scale, rounded to the activation dtype (exact
// except an fp16 overflow of 2 s).  Per scale group the table {S0 = s | rnd(2s) << 16,
// S1 = -s | -rnd(2s) << 16}; a 256-entry LDS table (4 KB, `kSel1Entries`) maps a code to
// four v_perm_b32 selector words (selector byte 12 gives the zero bytes).
template <int DT, int GS>
struct RootRowDecoder {
    static_assert(GS == 8 || GS == 16 || GS == 32 || GS == 64, "1-bit group size 8..64");
    static constexpr int kLoads = 2;
    uint32_t c;       // the half-row's 4 codes (32 weights)
    uint2 sc;         // its scales, as Bit2RowDecoder
    uint4 sel[4];     // selector words of pieces 0..3
    uint2 val[4];     // value words of pieces 0..3
    const char* tab;
    uint32_t vo_code, vo_scale;
    __amdgpu_buffer_rsrc_t pr, sr;
    __device__ __forceinline__ void load(int64_t k0) {
        c = __builtin_amdgcn_raw_buffer_load_b32(pr, vo_code, uniform_offset(k0 / 8), 0);
        const int so = uniform_offset(k0 * 2 / GS);
        if constexpr (GS == 8) {
            const auto u = __builtin_amdgcn_raw_buffer_load_b64(sr, vo_scale, so, 0);
            sc = make_uint2(u[0], u[1]);
        } else if constexpr (GS == 16) {
            sc = make_uint2(__builtin_amdgcn_raw_buffer_load_b32(sr, vo_scale, so, 0), 0u);
        } else {
            sc = make_uint2(__builtin_amdgcn_raw_buffer_load_b16(sr, vo_scale, so, 0), 0u);
        }
    }
    __device__ __forceinline__ void prep() {
#pragma unroll
        for (int p = 0; p < 4; ++p)
            sel[p] = *reinterpret_cast<const uint4*>(tab + 16u * ((c >> (8 * p)) & 0xFFu));
        if constexpr (GS == 8) {
            val[0] = values1<DT>(sc.x);
            val[1] = values1<DT>(sc.x >> 16);
            val[2] = values1<DT>(sc.y);
            val[3] = values1<DT>(sc.y >> 16);
        } else if constexpr (GS == 16) {
            val[0] = val[1] = values1<DT>(sc.x);
            val[2] = val[3] = values1<DT>(sc.x >> 16);
        } else {
            val[0] = val[1] = val[2] = val[3] = values1<DT>(sc.x);
        }
    }
    __device__ __forceinline__ uint4 piece(int p) const {
        const uint32_t s0 = val[p].x, s1 = val[p].y;
        return make_uint4(__builtin_amdgcn_perm(s0, s1, sel[p].x),
                          __builtin_amdgcn_perm(s0, s1, sel[p].y),
                          __builtin_amdgcn_perm(s0, s1, sel[p].z),
                          __builtin_amdgcn_perm(s0, s1, sel[p].w));
    }
    __device__ __forceinline__ void store(int p, char* tile, uint32_t wrow, int hf) const {
        *reinterpret_cast<uint4*>(tile + swz(wrow, 4u * hf + p)) = piece(p);
    }
};

// ---- backward-dX decoders: gx[M, K] = gy[M, N] . W[N, K] runs the same MFMA loop with the
// weight tile transposed: tile row = output column k, piece = 8 consecutive reduction rows
// n.  Thread pair (2b, 2b + 1) owns the 8 x 8 block b of the step's 64 x BN slice: rows
// n = 8 (b % 8) + 4 h .. + 3 (h = the thread's parity), columns k = 8 (b / 8) .. + 7.  Each
// thread expands the code of its 4 rows into 4 rows of 8 weights (dwords of k pairs), then
// v_perm_b32 transposes them into 8 columns of 4 weights (dwords of n pairs) written as
// 8-byte halves of the tile's pieces.

struct BwdBlock {
    uint32_t rows;   // 8 (b % 8) + 4 h: first of the thread's 4 weight rows in the step
    uint32_t col;    // 8 (b / 8): first tile column (output k) of the block
    uint32_t piece;  // b % 8
    uint32_t hoff;   // 8 h: byte offset inside the piece
};

__device__ __forceinline__ BwdBlock bwd_block(int tid) {
    const uint32_t b = (uint32_t)tid >> 1;
    BwdBlock k;
    k.piece = b & 7u;
    k.rows = 8u * k.piece + 4u * ((uint32_t)tid & 1u);
    k.col = 8u * (b >> 3);
    k.hoff = 8u * ((uint32_t)tid & 1u);
    return k;
}

// Writes columns 2p and 2p + 1 of a thread pair's 8 x 8 block (r[row][dword of k pairs], the
// thread's 4 rows) as dwords of n pairs.  Paired: each thread of the pair builds its 8-byte
// half of both columns, swaps one with its neighbour lane, and writes the whole 16-byte piece
// of column 2p + h (rows 0-3 from the even lane, 4-7 from the odd one); unpaired: each thread
// writes its halves of both columns.  Measured (backward dX, bf16, prefill shapes): paired
// ternary +1.6%, 2-bit +0.5%, 1-bit -4% (its kernel then needs 253 VGPRs); 1-bit stays unpaired.
template <bool Paired>
__device__ __forceinline__ void bwd_store_cols(const uint32_t (&r)[4][4], int p, char* tile,
                                               const BwdBlock& bk) {
    if constexpr (Paired) {
        const bool odd = bk.hoff != 0;
        const uint32_t selk = odd ? 0x07060302u : 0x05040100u;  // column 2p + h: kept
        const uint32_t sels = odd ? 0x05040100u : 0x07060302u;  // column 2p + 1 - h: sent
        const uint32_t k0 = __builtin_amdgcn_perm(r[1][p], r[0][p], selk);
        const uint32_t k1 = __builtin_amdgcn_perm(r[3][p], r[2][p], selk);
        const uint32_t s0 = __builtin_amdgcn_perm(r[1][p], r[0][p], sels);
        const uint32_t s1 = __builtin_amdgcn_perm(r[3][p], r[2][p], sels);
        // quad_perm [1, 0, 3, 2]: the neighbour lane's value
        const uint32_t o0 = (uint32_t)__builtin_amdgcn_mov_dpp((int)s0, 0xB1, 0xF, 0xF, false);
        const uint32_t o1 = (uint32_t)__builtin_amdgcn_mov_dpp((int)s1, 0xB1, 0xF, 0xF, false);
        const uint4 v = odd ? make_uint4(o0, o1, k0, k1) : make_uint4(k0, k1, o0, o1);
        *reinterpret_cast<uint4*>(tile + swz(bk.col + 2u * (uint32_t)p + (odd ? 1u : 0u), bk.piece)) = v;
    } else {
#pragma unroll
        for (int c2 = 0; c2 < 2; ++c2) {
            const int c = 2 * p + c2;
            const uint32_t sel = (c & 1) ? 0x07060302u : 0x05040100u;
            const uint32_t d0 = __builtin_amdgcn_perm(r[1][c >> 1], r[0][c >> 1], sel);
            const uint32_t d1 = __builtin_amdgcn_perm(r[3][c >> 1], r[2][c >> 1], sel);
            *reinterpret_cast<uint2*>(tile + swz(bk.col + (uint32_t)c, bk.piece) + bk.hoff) =
                make_uint2(d0, d1);
        }
    }
}

// One scale in the activation dtype as the AND word s | s << 16 | 0x80008000 (ternary masks).
template <int DT>
__device__ __forceinline__ uint32_t scale_word1(uint32_t s16) {
    uint32_t p;
    if constexpr (DT == kBF16) p = (uint32_t)__builtin_bit_cast(uint16_t, (__bf16)f16_bits_to_f32(s16 & 0xFFFFu));
    else p = s16 & 0xFFFFu;
    return (p | (p << 16)) | 0x80008000u;
}

// Ternary backward dX with the step's code bytes (and at BN = 256 its scale bytes) staged in
// LDS.  The 64 weight rows of a K step need BN * 3 / 16 code bytes and BN / 16 scale bytes
// each for the tile's BN output columns, fetched as pieces of BN / 16 bytes: three code
// pieces per row, then (BN = 256) one scale piece per row.  Each of the first 256 threads
// fetches one piece per step (at BN = 256 threads t and t + 256 fetch the same piece, so that
// every wave issues one load per step; at BN = 128 the fourth wave fetches nothing, from past
// the buffer's end) and writes it into a ring of step slots in LDS one step after the fetch.
// A thread then reads the two dwords that hold its row's 12-bit code (and its 16-bit scale)
// from LDS instead of issuing twelve byte loads per step; at BN = 128 the scales stay four
// 16-bit loads per thread (a staged scale slot would take the LDS that lets two workgroups
// share a CU).  The loop step that computes step s expands step s + 1, writes step
// s + kSlots and fetches step s + kSlots + 1, so a slot is rewritten one barrier after its
// last expansion.  Three slots at BN = 256 (2-3% faster than two there), two at BN = 128
// (the LDS of two workgroups per CU).
// The ring holds a step's rows in the order R = 16 (r % 4) + r / 4, so that the 16 rows
// 4 apart that one read instruction's lanes touch (a thread's rows are 4 apart from its
// neighbours') sit in consecutive ring rows, on distinct LDS banks; ring row R holds weight
// row bwd_ring_row(R) (measured: 3.9 bank-conflict cycles per LDS instruction with rows in
// order).  The fetching thread of ring position i loads the piece that belongs there, so
// the ring is filled in position order (as the LDS DMA writes it).
__device__ __forceinline__ uint32_t bwd_ring_row(uint32_t R) { return 4u * (R & 15u) + (R >> 4); }

template <int BN, int GS>
struct BwdStage {
    // scales staged as well at BN = 256 and group size 32 (one 16-byte piece per row)
    static constexpr bool kScales = BN == 256 && GS == 32;
    static constexpr uint32_t kCodeRow = BN * 3 / 16;   // code bytes per row and step
    static constexpr uint32_t kScaleRow = BN / 16;      // scale bytes per row and step
    static constexpr uint32_t kPiece = BN / 16;         // bytes per fetched piece
    static constexpr uint32_t kBytes = 64 * (kCodeRow + (kScales ? kScaleRow : 0));
    static constexpr int kSlots = BN == 256 ? 3 : 2;
    static_assert(kCodeRow == 3 * kPiece, "three code pieces per row");
};
constexpr uint32_t kBwdOob = 0x80000000u;  // a buffer offset past every operand: loads zeros

// One 16-byte-per-lane buffer->LDS load (a wave's 1 KB) at `dst`.  (Not a template: the host
// pass drops a kernel template that calls this builtin directly.)
__device__ __forceinline__ void bwd_stage_dma(char* dst, __amdgpu_buffer_rsrc_t r, uint32_t vo,
                                              int so) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void*)dst, 16,
                                             vo, so, 0, 0);
}

template <int DT, int BN, int GS>
struct TernaryBwdStagedDecoder {
    using St = BwdStage<BN, GS>;
    static_assert(BN == 256 || BN == 128, "16- or 8-byte pieces");
    static_assert(BN == 256 || St::kSlots == 2, "init fills two slots through registers");
    static constexpr int kLoads = St::kScales ? 1 : 5;
    static constexpr bool kStaged = true;
    using Piece = std::conditional_t<BN == 256, u32x4, u32x2>;
    uint32_t r[4][4];
    uint32_t vo_piece, rowbytes, srowbytes;  // this thread's piece of a step (step 0)
    bool scale_piece;                        // the piece holds scales (BN = 256, t >= 192)
    uint32_t rd_code, rd_shift, rd_scale;    // its own code's dwords and scale in a slot
    bool writer;                             // writes its piece to the ring
    Piece pend;                              // fetched piece of step `nl - 1`
    uint32_t sc[4], vo_scale[4];             // BN = 128: the scales of the thread's rows
    int nl;                                  // next step to fetch (relative to the first)
    int np;                                  // next step to expand
    int64_t k_first;
    char* ring;                              // St::kSlots slots of St::kBytes
    const char* lut;
    uint32_t slot;
    __amdgpu_buffer_rsrc_t pr, sr;
    BwdBlock bk;
    // (+16: the dword after a BN = 128 slot's last code row, which its last codes' reads touch)
    static constexpr uint32_t kRingBytes = St::kSlots * St::kBytes + 16;
    // block rows n and output columns k = n0 + bk.col .. + 7, as the unstaged decoder; the
    // tile's BN columns are codes 0 .. BN / 8 - 1 of a run of each row
    __device__ __forceinline__ void setup(int tid, int lane, int64_t n0, uint32_t rb, uint32_t srb,
                                          const char* table, char* ring_lds) {
        bk = bwd_block(tid);
        rowbytes = rb;
        srowbytes = srb;
        lut = table;
        slot = (uint32_t)(lane & (kLutSlots - 1)) * 8u;
        const uint32_t jj = bk.col / 8u;
        rd_code = St::kCodeRow * (bk.rows >> 2) + 4u * ((12u * jj) >> 5);
        rd_shift = (12u * jj) & 31u;
        rd_scale = 64u * St::kCodeRow + St::kScaleRow * (bk.rows >> 2) + 2u * (jj >> 2);
        const uint32_t t = (uint32_t)tid & 255u;
        // t >= 192 and tid < 256 are properties of the wave: taken from its (scalar) index,
        // the descriptor choice below stays scalar (a per-lane choice makes the compiler wrap
        // every load in a loop over the wave's distinct descriptors)
        const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
        scale_piece = St::kScales && (wv & 3) == 3;
        vo_piece = t >= 192u ? (St::kScales ? bwd_ring_row(t - 192u) * srb + (uint32_t)n0 / 16u : kBwdOob)
                             : bwd_ring_row(t / 3u) * rb + (uint32_t)n0 * 3u / 16u + St::kPiece * (t % 3u);
        writer = St::kScales ? wv < 4 : (wv & 3) < 3;
#pragma unroll
        for (int q = 0; q < 4; ++q)
            vo_scale[q] = (bk.rows + (uint32_t)q) * srb + 2u * (((uint32_t)n0 + bk.col) / GS);
        ring = ring_lds;
    }
    __device__ __forceinline__ Piece fetch(int t) const {
        const int64_t n0 = k_first + (int64_t)t * kBK;
        const __amdgpu_buffer_rsrc_t rs = scale_piece ? sr : pr;
        const int so = uniform_offset(n0 * (scale_piece ? srowbytes : rowbytes));
        if constexpr (BN == 256) return __builtin_amdgcn_raw_buffer_load_b128(rs, vo_piece, so, 0);
        else return __builtin_amdgcn_raw_buffer_load_b64(rs, vo_piece, so, 0);
    }
    __device__ __forceinline__ void load_scales(int64_t n0) {
        if constexpr (!St::kScales) {
            const int ss = uniform_offset(n0 * srowbytes);
#pragma unroll
            for (int q = 0; q < 4; ++q)
                sc[q] = __builtin_amdgcn_raw_buffer_load_b16(sr, vo_scale[q], ss, 0);
        }
    }
    __device__ __forceinline__ void put(int t, const Piece& v) const {
        char* dst = ring + (t % St::kSlots) * St::kBytes + St::kPiece * (threadIdx.x & 255u);
        if (writer) {
            if constexpr (BN == 256) *reinterpret_cast<uint4*>(dst) = make_uint4(v[0], v[1], v[2], v[3]);
            else *reinterpret_cast<uint2*>(dst) = make_uint2(v[0], v[1]);
        }
    }
    // the ring's first steps: BN = 256 loads them straight into the ring (buffer->LDS, 16
    // bytes per lane), BN = 128 through registers.  The caller waits for every load before
    // its barrier.
    __device__ __forceinline__ void init(int64_t k0) {
        k_first = k0;
        if constexpr (BN == 256) {
            load_scales(k0);  // scales not staged (group size other than 32): step 0's
            if (writer) {
                for (int t = 0; t < St::kSlots; ++t) {
                    const int64_t n0 = k0 + (int64_t)t * kBK;
                    bwd_stage_dma(ring + t * St::kBytes + 16u * ((threadIdx.x & 255u) & ~63u),
                                  scale_piece ? sr : pr, vo_piece,
                                  uniform_offset(n0 * (scale_piece ? srowbytes : rowbytes)));
                }
            }
        } else {
            const Piece v0 = fetch(0), v1 = fetch(1);
            load_scales(k0);
            put(0, v0);
            put(1, v1);
        }
        nl = St::kSlots;
        np = 0;
    }
    // write the piece fetched one step ago, fetch the next one (and the scales of step n0)
    __device__ __forceinline__ void load(int64_t n0) {
        if (nl > St::kSlots) put(nl - 1, pend);
        pend = fetch(nl);
        ++nl;
        load_scales(n0);
    }
    __device__ __forceinline__ void prep() {
        const char* sl = ring + (np % St::kSlots) * St::kBytes;
        ++np;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const uint32_t* cw = reinterpret_cast<const uint32_t*>(sl + 16u * St::kCodeRow * q + rd_code);
            const uint32_t code = __builtin_amdgcn_alignbit(cw[1], cw[0], rd_shift) & 0xFFFu;
            const uint32_t s16 =
                St::kScales ? *reinterpret_cast<const uint16_t*>(sl + 16u * St::kScaleRow * q + rd_scale)
                            : sc[q];
            const uint32_t z = (code << kCodeShift) | slot;
            const uint32_t h = __umulhi(z, kHiMagic);
            const uint2 ml = *reinterpret_cast<const uint2*>(lut + lo_addr_of(h, z));
            const uint2 mh = *reinterpret_cast<const uint2*>(lut + (h * kLutStride + slot));
            const uint32_t sw = scale_word1<DT>(s16);
            r[q][0] = ml.x & sw;
            r[q][1] = ml.y & sw;
            r[q][2] = mh.x & sw;
            r[q][3] = mh.y & sw;
        }
    }
    __device__ __forceinline__ void store(int p, char* tile, uint32_t, int) const {
        bwd_store_cols<true>(r, p, tile, bk);
    }
};

// B bytes (1, 2, 4, 8 or 16) from a buffer, in the low bytes of four dwords, and back to LDS.
template <int B>
__device__ __forceinline__ u32x4 piece_load(__amdgpu_buffer_rsrc_t r, uint32_t vo, int so) {
    static_assert(B == 1 || B == 2 || B == 4 || B == 8 || B == 16, "piece size");
    if constexpr (B == 16) {
        return __builtin_amdgcn_raw_buffer_load_b128(r, vo, so, 0);
    } else if constexpr (B == 8) {
        const u32x2 v = __builtin_amdgcn_raw_buffer_load_b64(r, vo, so, 0);
        return u32x4{v[0], v[1], 0u, 0u};
    } else if constexpr (B == 4) {
        return u32x4{__builtin_amdgcn_raw_buffer_load_b32(r, vo, so, 0), 0u, 0u, 0u};
    } else if constexpr (B == 2) {
        return u32x4{(uint32_t)__builtin_amdgcn_raw_buffer_load_b16(r, vo, so, 0), 0u, 0u, 0u};
    } else {
        return u32x4{(uint32_t)__builtin_amdgcn_raw_buffer_load_b8(r, vo, so, 0), 0u, 0u, 0u};
    }
}
template <int B>
__device__ __forceinline__ void piece_store(char* dst, const u32x4& v) {
    if constexpr (B == 16) *reinterpret_cast<uint4*>(dst) = make_uint4(v[0], v[1], v[2], v[3]);
    if constexpr (B == 8) *reinterpret_cast<uint2*>(dst) = make_uint2(v[0], v[1]);
    if constexpr (B == 4) *reinterpret_cast<uint32_t*>(dst) = v[0];
    if constexpr (B == 2) *reinterpret_cast<uint16_t*>(dst) = (uint16_t)v[0];
    if constexpr (B == 1) *reinterpret_cast<uint8_t*>(dst) = (uint8_t)v[0];
}

// 2-bit and 1-bit backward dX with the step's code and scale bytes staged in LDS, as the
// ternary staged decoder: the 64 weight rows of a K step need BN / 4 (2-bit) or BN / 8
// (1-bit) code bytes and 2 BN / GS scale bytes each for the tile's BN output columns; four
// threads share a row, each fetching a quarter of its codes and a quarter of its scales (one
// load of each per step; at BN = 256 threads t and t + 256 fetch the same pieces).  The
// pieces go into a two-slot ring one step after the fetch; each thread then reads its four
// rows' code bytes (two for 2-bit, one for 1-bit) and scales from LDS instead of issuing
// eight loads per step.
template <int DT, int BN, int FMT, int GS>
struct LowbitBwdStagedDecoder {
    static constexpr bool kTwoBit = FMT == kFmt2Bit;
    static constexpr uint32_t kCodeRow = kTwoBit ? BN / 4 : BN / 8;  // code bytes per row, step
    static constexpr uint32_t kScaleRow = 2 * BN / GS;               // scale bytes per row, step
    static constexpr int kCP = (int)kCodeRow / 4, kSP = (int)kScaleRow / 4;  // bytes per thread
    static constexpr uint32_t kCodeBytes = 64 * kCodeRow;
    static constexpr uint32_t kBytes = 64 * (kCodeRow + kScaleRow);
    static constexpr int kSlots = 2;
    static constexpr uint32_t kRingBytes = kSlots * kBytes;
    static constexpr int kLoads = 2;
    static constexpr bool kStaged = true;
    static_assert(kCP >= 4 && kCP <= 16 && kSP >= 1 && kSP <= 16, "piece sizes");
    // Rows are in ring order (bwd_ring_row) and, where a row is 32 or 64 bytes, its four
    // pieces are XOR-permuted by ring row, so that a read instruction's 16 consecutive ring
    // rows land on distinct LDS banks (64-byte rows would otherwise repeat every 4 rows).
    template <uint32_t ROW>
    static __device__ __forceinline__ uint32_t swz(uint32_t R) {
        constexpr uint32_t kShift = ROW >= 64 ? 2 : (ROW == 32 ? 3 : 4);
        return ((R & 15u) >> kShift) & 3u;
    }
    uint32_t r[4][4];
    uint32_t vo_code, vo_scale, rowbytes, srowbytes;  // this thread's pieces of step 0
    uint32_t rd_code, rd_scale;                       // its rows' code and scale bytes in a slot
    bool writer;
    u32x4 pc, ps;                                     // fetched pieces of step `nl - 1`
    int nl, np;
    int64_t k_first;
    char* ring;
    const char* tab;
    __amdgpu_buffer_rsrc_t pr, sr;
    BwdBlock bk;
    __device__ __forceinline__ void setup(int tid, int, int64_t n0, uint32_t rb, uint32_t srb,
                                          const char* table, char* ring_lds) {
        bk = bwd_block(tid);
        rowbytes = rb;
        srowbytes = srb;
        tab = table;
        const uint32_t t = (uint32_t)tid & 255u;
        // ring position t holds piece (t % 4) ^ swz of ring row t / 4
        const uint32_t R = t / 4u;
        vo_code = bwd_ring_row(R) * rb + (uint32_t)n0 / (kTwoBit ? 4u : 8u) +
                  (uint32_t)kCP * ((t % 4u) ^ swz<kCodeRow>(R));
        vo_scale = bwd_ring_row(R) * srb + 2u * ((uint32_t)n0 / GS) +
                   (uint32_t)kSP * ((t % 4u) ^ swz<kScaleRow>(R));
        // this thread's rows are bk.rows + q: ring rows 16 q + bk.rows / 4
        const uint32_t k = bk.rows >> 2;
        const uint32_t cb = bk.col / (kTwoBit ? 4u : 8u), sb = 2u * (bk.col / GS);
        rd_code = kCodeRow * k + (uint32_t)kCP * ((cb / kCP) ^ swz<kCodeRow>(k)) + cb % kCP;
        rd_scale = kCodeBytes + kScaleRow * k + (uint32_t)kSP * ((sb / kSP) ^ swz<kScaleRow>(k)) +
                   sb % kSP;
        writer = __builtin_amdgcn_readfirstlane(tid >> 6) < 4;  // a property of the wave
        ring = ring_lds;
    }
    __device__ __forceinline__ void fetch(int t, u32x4& c, u32x4& sv) const {
        const int64_t n0 = k_first + (int64_t)t * kBK;
        c = piece_load<kCP>(pr, vo_code, uniform_offset(n0 * rowbytes));
        sv = piece_load<kSP>(sr, vo_scale, uniform_offset(n0 * srowbytes));
    }
    __device__ __forceinline__ void put(int t, const u32x4& c, const u32x4& sv) const {
        char* sl = ring + (t % kSlots) * kBytes;
        const uint32_t i = threadIdx.x & 255u;
        if (writer) {
            piece_store<kCP>(sl + (uint32_t)kCP * i, c);
            piece_store<kSP>(sl + kCodeBytes + (uint32_t)kSP * i, sv);
        }
    }
    __device__ __forceinline__ void init(int64_t k0) {
        k_first = k0;
        u32x4 c0, s0, c1, s1;
        fetch(0, c0, s0);
        fetch(1, c1, s1);
        put(0, c0, s0);
        put(1, c1, s1);
        nl = kSlots;
        np = 0;
    }
    __device__ __forceinline__ void load(int64_t) {
        if (nl > kSlots) put(nl - 1, pc, ps);
        fetch(nl, pc, ps);
        ++nl;
    }
    __device__ __forceinline__ void prep() {
        const char* sl = ring + (np % kSlots) * kBytes;
        ++np;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const uint32_t s16 = *reinterpret_cast<const uint16_t*>(sl + rd_scale + 16u * kScaleRow * q);
            if constexpr (kTwoBit) {
                const uint32_t cw = *reinterpret_cast<const uint16_t*>(sl + rd_code + 16u * kCodeRow * q);
                const uint2 v = values2<DT>(s16);
                const uint2 a = *reinterpret_cast<const uint2*>(tab + 8u * (cw & 0xFFu));
                const uint2 b = *reinterpret_cast<const uint2*>(tab + 8u * (cw >> 8));
                r[q][0] = __builtin_amdgcn_perm(v.x, v.y, a.x);
                r[q][1] = __builtin_amdgcn_perm(v.x, v.y, a.y);
                r[q][2] = __builtin_amdgcn_perm(v.x, v.y, b.x);
                r[q][3] = __builtin_amdgcn_perm(v.x, v.y, b.y);
            } else {
                const uint32_t cd = *reinterpret_cast<const uint8_t*>(sl + rd_code + 16u * kCodeRow * q);
                const uint2 v = values1<DT>(s16);
                const uint4 e = *reinterpret_cast<const uint4*>(tab + 16u * cd);
                r[q][0] = __builtin_amdgcn_perm(v.x, v.y, e.x);
                r[q][1] = __builtin_amdgcn_perm(v.x, v.y, e.y);
                r[q][2] = __builtin_amdgcn_perm(v.x, v.y, e.z);
                r[q][3] = __builtin_amdgcn_perm(v.x, v.y, e.w);
            }
        }
    }
    __device__ __forceinline__ void store(int p, char* tile, uint32_t, int) const {
        bwd_store_cols<kTwoBit>(r, p, tile, bk);
    }
};

// Decoders that stage their codes through an LDS ring (declare kStaged).
template <typename D, typename = void>
struct IsStaged : std::false_type {};
template <typename D>
struct IsStaged<D, std::void_t<decltype(D::kStaged)>> : std::bool_constant<D::kStaged> {};
template <typename D, typename = void>
struct RingBytes : std::integral_constant<uint32_t, 16> {};
template <typename D>
struct RingBytes<D, std::void_t<decltype(D::kRingBytes)>>
    : std::integral_constant<uint32_t, D::kRingBytes> {};

// One K step (64) of the wave's block.
//   1. sub-step 0 on fragments already in registers (a0/b0) while sub-step 1's are read,
//      then the next step's X tile load is issued (issue_x);
//   2. the decoder's table reads for this thread's half row of the NEXT step's weights
//      (their codes arrived a full step ago), then its codes are re-armed with those of the
//      step after;
//   3. sub-step 1; in its last four MFMA rows the next step's weight pieces are written to
//      the other LDS buffer.
template <int DT, int TM, int TN, typename Dec, typename IssueX>
__device__ __forceinline__ void kstep(const char* xt, const char* wt, const FragLane& fl,
                                      uint4 (&a0)[TM], uint4 (&b0)[TN], uint4 (&a1)[TM],
                                      uint4 (&b1)[TN], Dec& dec, char* wt_next, uint32_t wrow,
                                      int half, f32x4 (&acc)[TM][TN], int64_t k_reload,
                                      const IssueX& issue_x) {
    const char* pa1 = xt + fl.a[1];
    const char* pb1 = wt + fl.b[1];
#pragma unroll
    for (int j = 0; j < TN; ++j) b1[j] = *reinterpret_cast<const uint4*>(pb1 + 2048 * j);
#pragma unroll
    for (int i = 0; i < TM; ++i) {
        mma_row<DT, TN>(a0[i], b0, acc[i]);
        a1[i] = *reinterpret_cast<const uint4*>(pa1 + 2048 * i);
    }
    // every read of this step's X tile is issued: the next X tile may now be loaded into
    // the other buffer without the compiler holding a later read of this one behind it
    issue_x();
    dec.prep();
    dec.load(k_reload);
#pragma unroll
    for (int i = 0; i < TM; ++i) {
        mma_row<DT, TN>(a1[i], b1, acc[i]);
        if (i >= TM - 4) {  // the table reads were issued TM - 4 MFMA rows earlier
            const int p = i - (TM - 4);
            dec.store(p, wt_next, wrow, half);
        }
    }
}

// s_waitcnt vmcnt(N) (fields vmcnt[3:0] and [15:14]; expcnt and lgkmcnt left alone):
// all but the N newest loads have completed.
template <int N>
__device__ __forceinline__ void vm_wait_le() {
    static_assert(N >= 0 && N < 64, "vmcnt holds 6 bits");
    __builtin_amdgcn_s_waitcnt(0x0F70 | (N & 15) | ((N >> 4) << 14));
}

// FMT: kFmtTernary (group size GS2 = 16, 32 or 64), kFmt2Bit or kFmtRoot (GS2 = 8 .. 64).  BWD = false:
// y[M, N] = x[M, K] . W[N, K]^T + bias; BWD = true: y[M, K] = x[M, N] . W[N, K] (backward
// dX; x is grad_y, bias unused).  The weight matrix is W[N, K] in both.
template <int DT, typename C, int FMT, int GS2, bool BWD>
__global__ __launch_bounds__(C::THREADS) void gemm_mfma_kernel(
    const void* __restrict__ x, const uint8_t* __restrict__ packed,
    const uint16_t* __restrict__ scales, const void* __restrict__ bias, void* __restrict__ y,
    float* __restrict__ part, int splits, int64_t M, int64_t N, int64_t K, LoraEp lora) {
    constexpr bool kTernary = FMT == kFmtTernary;
    const int64_t NO = BWD ? K : N;  // output columns
    const int64_t R = BWD ? N : K;   // reduction length (row length of x)
    __shared__ uint4 lut_storage[kTernary ? kLutStorageU4
                                          : (FMT == kFmt2Bit ? kSel2Entries / 2 : kSel1Entries)];
    __shared__ __attribute__((aligned(16))) char xs[2][C::XTILE];
    __shared__ __attribute__((aligned(16))) char ws[2][C::WTILE];
    constexpr int kTM = C::TM, kTN = C::TN;

    if constexpr (kTernary) fill_lut<C::THREADS>(lut_storage, kLutMasks);
    else if constexpr (FMT == kFmt2Bit) fill_sel2(reinterpret_cast<uint2*>(lut_storage), C::THREADS);
    else fill_sel1<C::THREADS>(lut_storage);

    // ---- tile assignment: contiguous tile range per XCD, M-grouped within it
    const int64_t tm_n = (M + C::BM - 1) / C::BM, tn_n = (NO + C::BN - 1) / C::BN;
    const int64_t tiles = tm_n * tn_n;
    // K split: workgroup blockIdx.x runs K steps [s_begin, s_end) of tile blockIdx.x % tiles
    const int split = (int)(blockIdx.x / (uint32_t)tiles);
    const int64_t bid = blockIdx.x - (int64_t)split * tiles;
    const int64_t per_xcd = (tiles + kXcds - 1) / kXcds;
    const int64_t xcd = bid % kXcds, slot_in = bid / kXcds;
    int64_t t = xcd * per_xcd + slot_in;
    if (per_xcd * kXcds != tiles) {
        // grid not a multiple of the XCD count: fall back to the plain order
        t = bid;
    }
    if (t >= tiles) return;
    // M tiles per group: fewer on wide forward outputs (gate/up, 56 column tiles at 256: a
    // group of 4 x 56 tiles is what an XCD's 32 CUs work through in about seven waves).
    // Measured on the prefill cases, 8 -> 4 for every shape: gate/up M = 8192 +3.6%, q/o
    // M = 2048 -5%, k/v M = 8192 -3.5%; for wide outputs only: +1% over the 12 cases, the
    // backward dX (wide for down) -0.6%, so it keeps 8.
    const int64_t gm = (!BWD && tn_n >= kGroup4FromTn) ? 4 : kGroupM;
    const int64_t group = t / (gm * tn_n);
    const int64_t first_m = group * gm;
    const int64_t gsize = (tm_n - first_m) < gm ? (tm_n - first_m) : gm;
    const int64_t tm = first_m + (t % (gm * tn_n)) % gsize;
    const int64_t tn = (t % (gm * tn_n)) / gsize;
    const int64_t m0 = tm * C::BM, n0 = tn * C::BN;

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int g = lane >> 4, i16 = lane & 15;
    const uint32_t arow0 = (uint32_t)C::WM * (uint32_t)(wave / C::WAVES_N);
    const uint32_t brow0 = (uint32_t)C::WN * (uint32_t)(wave % C::WAVES_N);

    const __amdgpu_buffer_rsrc_t xr = __builtin_amdgcn_make_buffer_rsrc(
        (void*)x, (short)0, (int)(M * R * 2), kRsrcWord3);
    const uint32_t rowbytes = kTernary ? (uint32_t)(K * 3 / 16)
                                       : (FMT == kFmt2Bit ? (uint32_t)(K / 4) : (uint32_t)(K / 8));
    const uint32_t srowbytes = (uint32_t)(K * 2 / GS2);
    const __amdgpu_buffer_rsrc_t pr = __builtin_amdgcn_make_buffer_rsrc(
        (void*)packed, (short)0, (int)(N * rowbytes), kRsrcWord3);
    const __amdgpu_buffer_rsrc_t sr = __builtin_amdgcn_make_buffer_rsrc(
        (void*)scales, (short)0, (int)(N * srowbytes), kRsrcWord3);
    const uint32_t wrow = (uint32_t)tid >> 1;  // this thread's weight row in the tile
    const int half = tid & 1;                   // ... and which half of its K step
    const uint32_t vo_code = (uint32_t)(n0 + wrow) * rowbytes;
    const uint32_t vo_scale = (uint32_t)(n0 + wrow) * srowbytes;
    const char* lut = reinterpret_cast<const char*>(lut_storage) + (kTernary ? kLutBaseOffset : 0);
    using FwdDec = std::conditional_t<
        kTernary, TernaryRowDecoder<DT, GS2>,
        std::conditional_t<FMT == kFmt2Bit, Bit2RowDecoder<DT, GS2>, RootRowDecoder<DT, GS2>>>;
    using BwdDec = std::conditional_t<kTernary, TernaryBwdStagedDecoder<DT, C::BN, GS2>,
                                      LowbitBwdStagedDecoder<DT, C::BN, FMT, GS2>>;
    using Dec = std::conditional_t<BWD, BwdDec, FwdDec>;
    constexpr bool kStagedDec = IsStaged<Dec>::value;
    __shared__ __attribute__((aligned(16))) char dec_ring[RingBytes<Dec>::value];
    Dec dec;
    dec.pr = pr;
    dec.sr = sr;
    if constexpr (kStagedDec) {
        dec.setup(tid, lane, n0, rowbytes, srowbytes, lut, dec_ring);
    } else if constexpr (kTernary) {
        dec.lut = lut;
        dec.slot = (uint32_t)(lane & (kLutSlots - 1)) * 8u;
        dec.vo_code = vo_code;
        dec.vo_scale = vo_scale;
        dec.half = half;
    } else {
        dec.tab = lut;
        dec.vo_code = vo_code + (FMT == kFmt2Bit ? 8u : 4u) * (uint32_t)half;
        // scale bytes of the half row: GS 8: 4 scales, 16: 2, 32: 1; GS 64: the step's one
        dec.vo_scale = vo_scale + (GS2 < 64 ? (uint32_t)half * (64u / GS2) : 0u);
    }

    f32x4 acc[kTM][kTN];
#pragma unroll
    for (int i = 0; i < kTM; ++i)
#pragma unroll
        for (int j = 0; j < kTN; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

    const int64_t steps = R / kBK;
    const int64_t s_begin = steps * split / splits, s_end = steps * (split + 1) / splits;
    const int64_t k_begin = s_begin * kBK;
    // Codes run one K step ahead of the weight tile being decoded, which runs one step
    // ahead of the MFMAs.  Branch-free body: loads past the last step fetch bytes past the
    // operands (zeros, or the next row's data) into buffers that are never read.
    load_x_tile(xs[0], xr, m0, k_begin, R, wave, lane, C::XLOADS);
    if constexpr (kStagedDec) {
        dec.init(k_begin);
        vm_wait_le<0>();  // the ring's first three steps have landed
    } else {
        dec.load(k_begin);
    }
    __syncthreads();  // table (and the staged decoder's first steps) ready
    dec.prep();
#pragma unroll
    for (int p = 0; p < 4; ++p) dec.store(p, ws[0], wrow, half);
    dec.load(k_begin + kBK);
    __builtin_amdgcn_s_waitcnt(0x0F70);
    __syncthreads();

    const FragLane fl = frag_lane(arow0, brow0, g, i16);
    uint4 a0[kTM], b0[kTN], a1[kTM], b1[kTN];
    load_frags(xs[0], ws[0], fl, 0, a0, b0);
    for (int64_t s = s_begin; s < s_end; ++s) {
        const int cur = (int)((s - s_begin) & 1), nxt = cur ^ 1;
        char* xn = xs[nxt];
        const int64_t kx = (s + 1) * kBK;
        // forward: the step's MFMA sections run at raised wave priority, so that of the two
        // waves on a SIMD the one with MFMAs to issue goes first while the other waits on
        // LDS (+2.8% on the prefill cases; the backward dX measured -0.7% with per-thread weight
        // loads and +-0 with its staged rings, and keeps priority 0)
        if constexpr (!BWD) __builtin_amdgcn_s_setprio(1);
        kstep<DT, kTM, kTN>(xs[cur], ws[cur], fl, a0, b0, a1, b1, dec, ws[nxt], wrow, half,
                            acc, (s + 2) * kBK,
                            [&] { load_x_tile(xn, xr, m0, kx, R, wave, lane, C::XLOADS); });
        if constexpr (!BWD) __builtin_amdgcn_s_setprio(0);
        vm_wait_le<Dec::kLoads>();  // the X tile of step s+1 has landed; code loads may fly
        __syncthreads();
        load_frags(xs[nxt], ws[nxt], fl, 0, a0, b0);
        // all of the step's first fragment reads go out before its first MFMA (left to
        // itself the scheduler sinks each A read to its MFMA row and exposes its latency)
        __builtin_amdgcn_sched_barrier(0);
    }

    // ---- epilogue: lane (g, i16) holds rows 4g+q of column i16 of each 16x16 tile
    if (splits > 1) {  // fp32 partial sums of this K range: part[split][row][col]
        float* pp = part + (int64_t)split * split_stride(M, NO);
#pragma unroll
        for (int j = 0; j < kTN; ++j) {
            const int64_t col = n0 + brow0 + 16 * j + i16;
            if (col >= NO) continue;
#pragma unroll
            for (int i = 0; i < kTM; ++i) {
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const int64_t row = m0 + arow0 + 16 * i + 4 * g + q;
                    if (row < M) pp[row * NO + col] = acc[i][j][q];
                }
            }
        }
        return;
    }
#pragma unroll
    for (int j = 0; j < kTN; ++j) {
        const int64_t col = n0 + brow0 + 16 * j + i16;
        if (col >= NO) continue;
        const float bv = (!BWD && bias) ? load_as_f32<DT>(bias, col) : 0.f;
#pragma unroll
        for (int i = 0; i < kTM; ++i) {
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const int64_t row = m0 + arow0 + 16 * i + 4 * g + q;
                if (row < M) {
                    float v = acc[i][j][q] + bv;
                    if (!BWD) v += lora_term<DT>(lora, row, col);
                    store_from_f32<DT>(y, row * NO + col, v);
                }
            }
        }
    }
}

// y[m, n] = sum over the K splits of part[s][m][n] (+ bias[n]), rounded once to dtype.
template <int DT>
__global__ __launch_bounds__(256) void gemm_split_reduce_kernel(
    const float* __restrict__ part, int splits, const void* __restrict__ bias,
    void* __restrict__ y, int64_t M, int64_t N, LoraEp lora) {
    const int64_t MN = M * N, stride = split_stride(M, N);
    const int64_t i4 = ((int64_t)blockIdx.x * 256 + threadIdx.x) * 4;
    if (i4 >= MN) return;
    if (i4 + 4 <= MN) {
        float4 a = *reinterpret_cast<const float4*>(part + i4);
        for (int s = 1; s < splits; ++s) {
            const float4 b = *reinterpret_cast<const float4*>(part + (int64_t)s * stride + i4);
            a.x += b.x; a.y += b.y; a.z += b.z; a.w += b.w;
        }
        const float v[4] = {a.x, a.y, a.z, a.w};
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int64_t i = i4 + e;
            const float bv = bias ? load_as_f32<DT>(bias, i % N) : 0.f;
            store_from_f32<DT>(y, i, v[e] + bv + lora_term<DT>(lora, i / N, i % N));
        }
    } else {
        for (int64_t i = i4; i < MN; ++i) {
            float a = 0.f;
            for (int s = 0; s < splits; ++s) a += part[(int64_t)s * stride + i];
            const float bv = bias ? load_as_f32<DT>(bias, i % N) : 0.f;
            store_from_f32<DT>(y, i, a + bv + lora_term<DT>(lora, i / N, i % N));
        }
    }
}

bool gemm_mfma_supported(const void* x, const uint8_t* packed, const uint16_t* scales,
                         int64_t M, int64_t N, int64_t K, int64_t gs, int dt, int fmt,
                         bool bwd) {
    if (dt != kBF16 && dt != kF16) return false;
    if (M < 1 || N < 1 || K < kBK || K % kBK != 0) return false;
    if (bwd && N % kBK != 0) return false;  // the backward reduces over N
    const int64_t R = bwd ? N : K;
    if (fmt == kFmtTernary ? (gs != 16 && gs != 32 && gs != 64)
                           : (gs != 8 && gs != 16 && gs != 32 && gs != 64))
        return false;
    if (fmt != kFmtTernary && fmt != kFmt2Bit && fmt != kFmtRoot) return false;
    if (((uintptr_t)x & 15u) || ((uintptr_t)packed & 7u) || ((uintptr_t)scales & 7u))
        return false;
    // 32-bit buffer offsets: the activation matrix and the weight buffers (plus one tile
    // of padding rows) must stay below 2^31 bytes
    const int64_t rowbytes = fmt == kFmtTernary ? K * 3 / 16 : (fmt == kFmt2Bit ? K / 4 : K / 8);
    const int64_t srowbytes = K * 2 / gs;
    if ((M + CfgLarge::BM) * R * 2 >= (1ll << 31) || (N + CfgLarge::BN) * rowbytes >= (1ll << 31) ||
        (N + CfgLarge::BN) * srowbytes >= (1ll << 31))
        return false;
    return true;
}

// Grids of large tiles that leave CUs idle (under about one workgroup per CU) run the
// small-tile configuration, which has four times the tiles and two workgroups per CU.

template <int DT, typename C, int FMT, int GS2, bool BWD>
static hipError_t launch_cfg(const void* x, const uint8_t* packed, const uint16_t* scales,
                             const void* bias, void* y, float* part, int splits, int64_t M,
                             int64_t N, int64_t K, hipStream_t stream, const LoraEp& lora) {
    const int64_t NO = BWD ? K : N;
    const int64_t tiles = ((M + C::BM - 1) / C::BM) * ((NO + C::BN - 1) / C::BN);
    if (tiles * splits > 0x7FFFFFFF) return hipErrorInvalidValue;
    hipLaunchKernelGGL((gemm_mfma_kernel<DT, C, FMT, GS2, BWD>), dim3((unsigned)(tiles * splits)),
                       dim3(C::THREADS), 0, stream, x, packed, scales, bias, y, part, splits, M,
                       N, K, lora);
    if (splits == 1) return hipGetLastError();
    const int64_t groups = (M * NO + 1023) / 1024;
    hipLaunchKernelGGL((gemm_split_reduce_kernel<DT>), dim3((unsigned)groups), dim3(256), 0,
                       stream, part, splits, BWD ? nullptr : bias, y, M, NO,
                       BWD ? LoraEp{} : lora);
    return hipGetLastError();
}

// Tile configuration and K split of a launch.
//  * Grids of at least 192 large tiles: large tiles, unsplit.
//  * Smaller grids: large tiles split over K towards one workgroup per CU, if every split
//    keeps at least kMinLargeSplitSteps K steps and the split grid still covers three
//    quarters of the CUs;
//  * otherwise small tiles, split over K towards two workgroups per CU (the small
//    configuration's residency), at least kMinSplitSteps K steps per split (8: at 4 the
//    fp32 partials of the k/v shape at M = 512 cost more than the extra workgroups gain;
//    16 for the backward dX, whose k/v shape at M = 512 runs 12% faster unsplit).
// The fp32 partial sums of a split stay under kSplitBytesMax.
constexpr int kMaxSplits = 16;
constexpr int64_t kMinSplitSteps = 8;
constexpr int64_t kMinSplitStepsBwd = 16;
constexpr int64_t kMinLargeSplitSteps = 16;
constexpr int64_t kSplitBytesMax = 256ll << 20;
constexpr int64_t kLargeTargetWgs = 256;
constexpr int64_t kLargeMinWgs = 192;

static int64_t splits_for(int64_t tiles, int64_t target, int64_t min_steps, int64_t M,
                          int64_t N, int64_t K) {
    int64_t s = (target + tiles / 2) / tiles;
    if (s > kMaxSplits) s = kMaxSplits;
    if (s > (K / kBK) / min_steps) s = (K / kBK) / min_steps;
    while (s > 1 && s * split_stride(M, N) * 4 > kSplitBytesMax) --s;
    return s < 1 ? 1 : s;
}

GemmChoice gemm_mfma_choice(int64_t M, int64_t N, int64_t K, bool bwd) {
    const int64_t large = ((M + CfgLarge::BM - 1) / CfgLarge::BM) *
                          ((N + CfgLarge::BN - 1) / CfgLarge::BN);
    if (large >= 192) return GemmChoice{false, 1};
    const int64_t sl = splits_for(large, kLargeTargetWgs, kMinLargeSplitSteps, M, N, K);
    if (large * sl >= kLargeMinWgs) return GemmChoice{false, (int)sl};
    const int64_t tiles = ((M + CfgSmall::BM - 1) / CfgSmall::BM) *
                          ((N + CfgSmall::BN - 1) / CfgSmall::BN);
    return GemmChoice{true,
                      (int)splits_for(tiles, 512,
                                      bwd ? kMinSplitStepsBwd : kMinSplitSteps, M, N, K)};
}

template <int DT, typename C, bool BWD>
static hipError_t launch_fmt(const void* x, const uint8_t* packed, const uint16_t* scales,
                             const void* bias, void* y, float* part, int splits, int64_t M,
                             int64_t N, int64_t K, int64_t gs, int fmt, hipStream_t stream,
                             const LoraEp& lora) {
    if (fmt == kFmtTernary) {
        switch (gs) {
        case 16:
            return launch_cfg<DT, C, kFmtTernary, 16, BWD>(x, packed, scales, bias, y, part, splits,
                                                          M, N, K, stream, lora);
        case 32:
            return launch_cfg<DT, C, kFmtTernary, 32, BWD>(x, packed, scales, bias, y, part, splits,
                                                          M, N, K, stream, lora);
        case 64:
            return launch_cfg<DT, C, kFmtTernary, 64, BWD>(x, packed, scales, bias, y, part, splits,
                                                          M, N, K, stream, lora);
        default:
            return hipErrorInvalidValue;
        }
    }
    if (fmt == kFmtRoot) {
        switch (gs) {
        case 8:
            return launch_cfg<DT, C, kFmtRoot, 8, BWD>(x, packed, scales, bias, y, part, splits, M, N,
                                                  K, stream, lora);
        case 16:
            return launch_cfg<DT, C, kFmtRoot, 16, BWD>(x, packed, scales, bias, y, part, splits, M, N,
                                                   K, stream, lora);
        case 32:
            return launch_cfg<DT, C, kFmtRoot, 32, BWD>(x, packed, scales, bias, y, part, splits, M, N,
                                                   K, stream, lora);
        case 64:
            return launch_cfg<DT, C, kFmtRoot, 64, BWD>(x, packed, scales, bias, y, part, splits, M, N,
                                                   K, stream, lora);
        default:
            return hipErrorInvalidValue;
        }
    }
    switch (gs) {
    case 8:
        return launch_cfg<DT, C, kFmt2Bit, 8, BWD>(x, packed, scales, bias, y, part, splits, M, N, K,
                                              stream, lora);
    case 16:
        return launch_cfg<DT, C, kFmt2Bit, 16, BWD>(x, packed, scales, bias, y, part, splits, M, N, K,
                                               stream, lora);
    case 32:
        return launch_cfg<DT, C, kFmt2Bit, 32, BWD>(x, packed, scales, bias, y, part, splits, M, N, K,
                                               stream, lora);
    case 64:
        return launch_cfg<DT, C, kFmt2Bit, 64, BWD>(x, packed, scales, bias, y, part, splits, M, N, K,
                                               stream, lora);
    default:
        return hipErrorInvalidValue;
    }
}

hipError_t launch_gemm_mfma(const void* x, const uint8_t* packed, const uint16_t* scales,
                            const void* bias, void* y, float* part, GemmChoice c, int64_t M,
                            int64_t N, int64_t K, int dt, hipStream_t stream, int64_t gs,
                            int fmt, bool bwd, const LoraEp& lora) {
    if (c.splits < 1 || (c.splits > 1 && !part)) return hipErrorInvalidValue;
    if (bwd) {
        if (dt == kBF16)
            return c.small ? launch_fmt<kBF16, CfgSmall, true>(x, packed, scales, bias, y, part,
                                                               c.splits, M, N, K, gs, fmt, stream, lora)
                           : launch_fmt<kBF16, CfgLarge, true>(x, packed, scales, bias, y, part,
                                                               c.splits, M, N, K, gs, fmt, stream, lora);
        return c.small ? launch_fmt<kF16, CfgSmall, true>(x, packed, scales, bias, y, part,
                                                          c.splits, M, N, K, gs, fmt, stream, lora)
                       : launch_fmt<kF16, CfgLarge, true>(x, packed, scales, bias, y, part,
                                                          c.splits, M, N, K, gs, fmt, stream, lora);
    }
    if (dt == kBF16)
        return c.small ? launch_fmt<kBF16, CfgSmall, false>(x, packed, scales, bias, y, part,
                                                            c.splits, M, N, K, gs, fmt, stream, lora)
                       : launch_fmt<kBF16, CfgLarge, false>(x, packed, scales, bias, y, part,
                                                            c.splits, M, N, K, gs, fmt, stream, lora);
    return c.small ? launch_fmt<kF16, CfgSmall, false>(x, packed, scales, bias, y, part, c.splits,
                                                       M, N, K, gs, fmt, stream, lora)
                   : launch_fmt<kF16, CfgLarge, false>(x, packed, scales, bias, y, part, c.splits,
                                                       M, N, K, gs, fmt, stream, lora);
}

}  // namespace ojx
