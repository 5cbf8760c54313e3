// e8t_internal.h -- launchers shared between the kernel files and the C ABI.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "e8t_device.h"

namespace ojx {

hipError_t launch_encode(const void* w, int wdt, int64_t numel, int64_t gs, uint8_t* packed,
                         uint16_t* scales, hipStream_t stream);

hipError_t launch_decode(const uint8_t* packed, const uint16_t* scales, int64_t numel, int64_t gs,
                         int odt, void* out, hipStream_t stream);

// 2-bit E8 codec (E8LatticePacker): gs a positive multiple of 8.
hipError_t launch_encode2(const void* w, int wdt, int64_t numel, int64_t gs, uint8_t* packed,
                          uint16_t* scales, hipStream_t stream);
hipError_t launch_decode2(const uint8_t* packed, const uint16_t* scales, int64_t numel,
                          int64_t gs, int odt, void* out, hipStream_t stream);

// 1-bit Root-E8 codec (RootE8LatticePacker): gs a positive multiple of 8.
hipError_t launch_encode1(const void* w, int wdt, int64_t numel, int64_t gs, uint8_t* codes,
                          uint16_t* scales, hipStream_t stream);
hipError_t launch_decode1(const uint8_t* codes, const uint16_t* scales, int64_t numel,
                          int64_t gs, int odt, void* out, hipStream_t stream);

// Conway-Sloane E8 projection (fp32 or fp64, nvec 8-vectors) and the QAT straight-through
// quantizer (fp32 weights).
// fwht_block32 of `blocks` contiguous 32-element blocks (dt: kF32, kF16, kBF16, kF64).
hipError_t launch_fwht32(const void* x, int dt, int64_t blocks, void* y, hipStream_t stream);
hipError_t launch_cs_project(const void* x, bool f64, int64_t nvec, void* out,
                             hipStream_t stream);
hipError_t launch_ste_quantize(const float* w, int64_t numel, float* out, hipStream_t stream);
// The same for dtype dt (kF32, kF64 for the projection, kF16, kBF16: every op rounded to the
// half type, as torch evaluates the reference on such tensors).
hipError_t launch_cs_project_dt(const void* x, int dt, int64_t nvec, void* out,
                                hipStream_t stream);
hipError_t launch_ste_quantize_dt(const void* w, int dt, int64_t numel, void* out,
                                  hipStream_t stream);

// Post-scaled decode GEMV of 2-bit (fmt 1, M <= 4) or 1-bit Root-E8 (fmt 2, M == 1) codes
// (bf16/fp16, K % 1024 == 0, gs in {8, 16, 32, 64}, 16-byte aligned buffers).
bool gemv2_supported(const void* x, const uint8_t* packed, const uint16_t* scales,
                     const void* y, int64_t M, int64_t N, int64_t K, int64_t gs, int dt, int fmt);
hipError_t launch_gemv2(const void* x, const uint8_t* packed, const uint16_t* scales,
                        const void* bias, void* y, int64_t M, int64_t N, int64_t K, int64_t gs,
                        int dt, hipStream_t stream, const LoraEp& lora, int fmt);

// Decode GEMV with the weights in the B operand for the ternary (fmt 0, gs 32), 2-bit (fmt 1)
// and 1-bit Root-E8 (fmt 2) formats: M <= 16, bf16/fp16, K % 256 == 0, gs in {8, 16, 32, 64},
// 16-byte aligned buffers.
bool gemv2m_supported(const void* x, const uint8_t* packed, const uint16_t* scales,
                      const void* y, int64_t M, int64_t N, int64_t K, int64_t gs, int dt,
                      int fmt);
hipError_t launch_gemv2m(const void* x, const uint8_t* packed, const uint16_t* scales,
                         const void* bias, void* y, int64_t M, int64_t N, int64_t K, int64_t gs,
                         int dt, hipStream_t stream, int fmt, const LoraEp& lora = LoraEp{});

// General tiled kernels: any M, N, K >= 1 (flat layout), any dtype; fmt selects the code
// format (0 ternary, 1 2-bit, 2 1-bit Root E8).
hipError_t launch_gemm_generic_fwd(const void* x, const uint8_t* packed, const uint16_t* scales,
                                   const void* bias, void* y, int64_t M, int64_t N, int64_t K,
                                   int64_t gs, int dt, hipStream_t stream, int fmt = 0,
                                   const LoraEp& lora = LoraEp{});
hipError_t launch_gemm_generic_bwd(const void* gy, const uint8_t* packed, const uint16_t* scales,
                                   void* gx, int64_t M, int64_t N, int64_t K, int64_t gs, int dt,
                                   hipStream_t stream, int fmt = 0);

}  // namespace ojx

namespace ojx {

// One linear of a (possibly grouped) decode-GEMV launch; same field order and types as
// ojx_e8t_gemv_job in include/ojasx_e8t.h.  Device pointers; flat layout with
// K % 256 == 0 and group size 32.
struct GemvJob {
    const void* x;            // [M, K] activations, or nullptr: the launch's x
    const uint8_t* packed;    // [N * K * 3 / 16]
    const uint16_t* scales;   // [N * K / 32] fp16 bits
    const void* bias;         // [N] or nullptr
    void* y;                  // output base, or nullptr: the launch's y
    int64_t N;
    int64_t K;
    int64_t y_col;            // first output column of this job in y
    int64_t y_ld;             // row stride of y in elements
    int64_t wg_begin;         // first workgroup of this job in the launch grid
    const float* lora_u;      // LoRA: scaling * (x @ A), fp32 [M, lora_r] (stride lora_ldu)
    const void* lora_b;       // LoRA up-projection [lora_r, N] in the activation dtype
    int64_t lora_r;           // adapter rank (0: none)
    int64_t lora_ldu;         // row stride of lora_u
    const void* lora_a;       // LoRA down-projection A [K, lora_r] (u is computed from it)
    float lora_scaling;
    int32_t reserved;
};

constexpr int kGemvInlineJobs = 4;

struct GemvLaunch {
    GemvJob inl[kGemvInlineJobs];  // used when jobs == nullptr
    const GemvJob* jobs;           // device array of njobs jobs, sorted by wg_begin
    const void* x;                 // default activations
    void* y;                       // default output
    int njobs;
    int M;
    int lora_inline;               // staged-tile kernel, one round per wave: jobs with an
                                   // adapter form u from lora_a themselves (lora_u unused)
};

// Grouped 2-bit or 1-bit decode GEMV (streaming kernel, fmt kFmt2Bit / kFmtRoot): 2-bit at
// M <= 4 with every K a multiple of 1024 runs post-scaled 1024-k rounds, otherwise B-operand
// 256-k rounds; R row tiles per workgroup.  Each job's tiles start a new workgroup.
struct Gemv2Plan {
    bool post;            // post-scaled form (M <= 4), else the B-operand form
    bool grouped_rounds;  // B-operand form: rounds fetched in load groups (every K % 1024 == 0)
    int R;                // row tiles per workgroup
};
Gemv2Plan gemv2_pick_grouped(int64_t total_tiles, int64_t M, bool k1024, int fmt);
int64_t gemv2_wgs_for(int64_t N, const Gemv2Plan& p);
hipError_t launch_gemv2_grouped(const GemvLaunch& a, const Gemv2Plan& p, int64_t wgs,
                                int64_t gs, int dt, int fmt, hipStream_t s);
bool gemv_shape_ok(int64_t N, int64_t K);
// Whether a staged-tile launch forms the adapters' u inside the launch: one round per wave
// (U == 1), one row tile per wave and per workgroup (rt == tpw == 1), rank-8 adapters with
// 16-byte aligned A.  The second form plans a per-linear launch of an [N, K] layer.
bool gemv_lora_inline_ok(int U, int rt, int tpw, int64_t rank, const void* lora_a);
bool gemv_tile_lora_inline_ok(int64_t M, int64_t N, int64_t K, int64_t rank,
                              const void* lora_a);
bool gemv_supported(const void* x, const uint8_t* packed, const uint16_t* scales, const void* y,
                    int64_t M, int64_t N, int64_t K, int64_t gs, int dt);
// Kernel variant of a decode-GEMV launch.
struct GemvPlan {
    bool wide;   // streaming kernel (one tile set per wave, full K) vs in-workgroup K split
    int R;       // 16-row tiles per wave
    int S;       // K split ways inside the workgroup (non-wide only)
    int W;       // waves per workgroup (wide only)
    int mmax;    // activation rows staged in LDS (wide only): 1, 4 (post-scaled) or 16
    int C;       // consecutive tile groups per workgroup (post-scaled kernel; else 1)
    bool split_ps;  // small-layer post-scaled kernel: one tile per workgroup, K split over waves
    bool tile;   // staged-tile kernel: U rounds per wave, tpw row tiles per workgroup, rt
    int U;       //   of them per wave
    int tpw;
    int rt;
};
GemvPlan gemv_pick(int64_t total_tiles, int64_t M);
// gemv_pick for a grouped launch, preferring the staged-tile kernel for launches of fewer
// than 4096 (M == 1) or 1024 (1 < M <= 4) row tiles
// when every job allows it (K % 1024 == 0, 16-byte aligned codes and scales; kmax the
// longest K).
GemvPlan gemv_pick_grouped(int64_t total_tiles, int64_t M, int64_t kmax, bool tile_ok);
int64_t gemv_wgs_for(int64_t N, const GemvPlan& p);
hipError_t launch_gemv(const GemvLaunch& a, const GemvPlan& p, int64_t wgs, int dt,
                       hipStream_t stream);

// Staged-tile decode GEMV (per-linear launches of small layers): 1 <= M <= 4, bf16/fp16,
// ternary codes with group size 32, K % 1024 == 0 up to K = 8192 (M = 1: 16384), 16-byte
// aligned buffers.  One workgroup per 16-row tile (wgs = the row tiles of the launch's
// jobs); Kmax the longest K of the jobs.
int gemv_tile_rounds(int64_t M, int64_t Kmax);
bool gemv_tile_supported(const void* x, const uint8_t* packed, const uint16_t* scales,
                         const void* y, int64_t M, int64_t N, int64_t K, int64_t gs, int dt);
hipError_t launch_gemv_tile(const GemvLaunch& a, int64_t tiles, int64_t Kmax, int dt,
                            hipStream_t stream, int64_t gs = 32);
// Row tiles per workgroup of a one-job staged-tile launch over `tiles` row tiles.
int gemv_tile_per_wg(int64_t M, int64_t tiles);

// Prefill MFMA GEMM: F16/BF16, K % 64 == 0; fmt 0 (ternary, group size 32), 1 (2-bit) or 2
// (1-bit Root E8), the last two with group size 8, 16, 32 or 64.
// bwd: the backward dX y[M, K] = x[M, N] . W[N, K] (also needs N % 64 == 0).
bool gemm_mfma_supported(const void* x, const uint8_t* packed, const uint16_t* scales,
                         int64_t M, int64_t N, int64_t K, int64_t gs, int dt, int fmt = 0,
                         bool bwd = false);
// Tile configuration and K splits of the prefill GEMM for a shape (splits 1 = none).  With
// splits > 1 the launch needs `part`, fp32 scratch of splits * split_stride(M, N) floats.
struct GemmChoice {
    bool small;  // 128 x 128 tiles (else 256 x 256)
    int splits;
};
GemmChoice gemm_mfma_choice(int64_t M, int64_t N, int64_t K, bool bwd);
__host__ __device__ inline int64_t split_stride(int64_t M, int64_t N) {
    return (M * N + 3) & ~(int64_t)3;  // 16-byte aligned per split
}
hipError_t launch_gemm_mfma(const void* x, const uint8_t* packed, const uint16_t* scales,
                            const void* bias, void* y, float* part, GemmChoice c, int64_t M,
                            int64_t N, int64_t K, int dt, hipStream_t stream, int64_t gs = 32,
                            int fmt = 0, bool bwd = false, const LoraEp& lora = LoraEp{});

// LoRA down-projection u[m, j] = scaling * sum_k x[m, k] A[k, j] (fp32 out, row stride ldu)
// for ranks 1 .. kLoraMaxRank; x and A in dtype dt.
constexpr int64_t kLoraMaxRank = 64;
hipError_t launch_lora_down(const void* x, const void* a, int64_t M, int64_t K, int64_t r,
                            float scaling, int dt, float* u, int64_t ldu, hipStream_t stream);
// Several adapters on the same x (up to kLoraDownItems per launch).
struct LoraDown {
    const void* a;   // [K, r] in dtype
    float* u;        // fp32 [M, r], row stride ldu
    int64_t r;
    int64_t ldu;
    float scaling;
};
constexpr int kLoraDownItems = 4;
hipError_t launch_lora_down(const void* x, int64_t M, int64_t K, int dt, const LoraDown* items,
                            int n, hipStream_t stream);

// Records `msg` as the calling thread's last error (ojx_e8t_last_error) and returns `code`.
int api_fail(int code, const char* msg);

// Bytes of fp32 K-split scratch a launch with choice `c` uses (0 when unsplit).
inline size_t gemm_split_bytes(const GemmChoice& c, int64_t M, int64_t out_cols) {
    return c.splits > 1 ? (size_t)c.splits * (size_t)split_stride(M, out_cols) * sizeof(float)
                        : 0;
}

}  // namespace ojx
