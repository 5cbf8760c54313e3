/*
 * ojasx_e8t.h -- C ABI of the MI355X (gfx950) ternary-E8 quantized-weight path.
 *
 * Shared library: ojasx-open-source-cuda_amd/lib/libojasx_e8t.so
 *
 * Plain pointers and sizes only.  Every pointer argument except `stream` is a
 * device pointer (HBM) on the current HIP device.  `stream` is a hipStream_t
 * (NULL = the null stream).  Each entry point enqueues its kernels on `stream`
 * and returns without synchronising; results are ready when the stream is.  The
 * library never allocates device memory: outputs and the scratch ("workspace") of the
 * fused GEMMs are the caller's.  A GEMM's workspace holds the fp32 partial sums of its
 * K split (prefill shapes whose tile grid is too small to fill the GPU); its size comes
 * from ojx_gemm_workspace_bytes, and a smaller one (or none) only lowers the split
 * count, down to the unsplit kernel, so results stay correct.  A workspace is in use
 * until the launch that received it has finished on its stream.  No mutable global
 * state beyond a per-device architecture check and a thread-local error message.
 *
 * Data layout (identical to the reference's buffers, so existing state_dicts load):
 *   packed  uint8 [padded * 3 / 16]   two 12-bit codes per 3 bytes, little-endian bit
 *                                      stream: code t occupies bits [12t, 12t+12)
 *                                      (ojasx2/math/lattice.py:375-383)
 *   scales  uint16 [padded / gs]       IEEE binary16 bit patterns, one per flat group of
 *                                      gs weights (lattice.py:355-356,384)
 *   padded  = numel rounded up to a multiple of gs (flat zero padding, lattice.py:351-353)
 *   A weight matrix W[N, K] is flattened row-major; element (n, k) is flat index n*K + k.
 *   When K % gs == 0 each row owns K*3/16 bytes and K/gs scales (streaming_e8.py:182-192).
 *
 * dtype codes: OJX_F32, OJX_F16, OJX_BF16 (activations, outputs, decoded weights).
 *
 * Return value: OJX_OK (0) or a negative OJX_E* status; ojx_e8t_last_error() gives the
 * message of the calling thread's last failure.
 */
#ifndef OJASX_E8T_H
#define OJASX_E8T_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum { OJX_F32 = 0, OJX_F16 = 1, OJX_BF16 = 2, OJX_F64 = 3 /* ojx_fwht32 only */ };

/* Weight formats (ojx_gemm_workspace_bytes): ternary E8 (1.5 bit), 2-bit E8, 1-bit Root E8. */
enum { OJX_FMT_TERNARY = 0, OJX_FMT_E8 = 1, OJX_FMT_ROOT = 2 };

enum {
    OJX_OK = 0,
    OJX_EINVAL = -1,  /* null pointer, negative or inconsistent size            */
    OJX_ELAYOUT = -2, /* group size / shape combination the op does not accept  */
    OJX_EDTYPE = -3,  /* unknown dtype code                                     */
    OJX_EHIP = -4,    /* HIP runtime or launch error                            */
    OJX_EDEVICE = -5  /* current device is not gfx950                           */
};

/* ABI version (major * 10000 + minor * 100 + patch). */
int ojx_e8t_version(void);

/* Message of the calling thread's last failed call ("" if none). */
const char* ojx_e8t_last_error(void);

/* Encoder.  Replaces TernaryE8LatticePacker.pack (ojasx2/math/lattice.py:338-384);
 * the reference's GPU route for it is a chain of ~25 ATen kernels, its streaming
 * caller is streaming_e8._pack_row_block (streaming_e8.py:112-123).
 *   w       [numel] weights of dtype w_dtype (F32, F16 or BF16; widened exactly to fp32)
 *   gs      group size; must be a positive multiple of 16 (the Python layer applies the
 *           reference's silent coercion to 16 first, lattice.py:346-347)
 *   packed  [padded*3/16] out,  scales [padded/gs] out (fp16 bits)
 * Bit-exact with the reference's CPU pack (ATen AVX2/AVX512 norm order). Inputs must be
 * finite. */
int ojx_e8t_encode(const void* w, int w_dtype, int64_t numel, int64_t gs, uint8_t* packed,
                   uint16_t* scales, void* stream);

/* Decoder.  Replaces TernaryE8LatticePacker.unpack (lattice.py:386-419).
 * Writes the first `numel` decoded weights in out_dtype:
 *   F32: coord * float(s16);  F16: coord * s16;  BF16: coord * bf16_rne(float(s16)).
 * Bit-exact with the reference. */
int ojx_e8t_decode(const uint8_t* packed, const uint16_t* scales, int64_t numel, int64_t gs,
                   int out_dtype, void* out, void* stream);

/* Workspace of a fused GEMM launch.  Writes to *bytes the device scratch that
 * ojx_{e8t,e8,e8r}_gemm_fwd (bwd = 0) or _gemm_bwd_dx (bwd = 1) uses for this shape at its
 * full K split, 0 when the launch needs none (every decode GEMV, M <= 16, and prefill grids
 * large enough to run unsplit).  fmt is an OJX_FMT_* code; (M, N, K) are the forward's
 * sizes (x [M, K], W [N, K]) for both directions.  Host-only: launches nothing.  No
 * counterpart in the reference, whose native ops allocate nothing but their output
 * (ojasx_math_bindings.cpp:432); it lets the caller own every byte this library touches. */
int ojx_gemm_workspace_bytes(int fmt, int bwd, int64_t M, int64_t N, int64_t K, int64_t gs,
                             int dtype, size_t* bytes);

/* Fused forward y[M,N] = x[M,K] . Wdeq[N,K]^T (+ bias[N]), fp32 accumulation, y in dtype.
 * Replaces fused_ternary_e8_gemm_fwd (ojasx2/math/csrc/ojasx_math_bindings.cpp:407-472,
 * schema at :594) and dispatch_tilelang_e8_gemm (ojasx2/tilelang_kernels.py:370-419);
 * called from _FusedE8GEMMFunction.forward (lattice.py:584-608).
 *   x, y, bias in `dtype`; bias may be NULL.  Wdeq follows the decoder's rule for `dtype`.
 *   Any K >= 1 (flat layout).  F16/BF16 with K % 256 == 0, gs in {16, 32, 64} and M <= 16
 *   run an MFMA decode GEMV; F16/BF16 with K % 64 == 0, gs in {16, 32, 64} and M > 16 the
 *   MFMA prefill GEMM; other shapes and F32 use a general tiled kernel.  Never declines.
 *   workspace: 16-byte aligned device scratch of workspace_bytes (NULL with 0 allowed),
 *   see ojx_gemm_workspace_bytes. */
int ojx_e8t_gemm_fwd(const void* x, const uint8_t* packed, const uint16_t* scales,
                     const void* bias, void* y, int64_t M, int64_t N, int64_t K, int64_t gs,
                     int dtype, void* workspace, size_t workspace_bytes, void* stream);

/* Allocation-free variant of ojx_e8t_gemm_fwd (same arguments minus the workspace, same
 * kernels and results).  No counterpart in the reference: it is for callers that cannot
 * allocate device memory (code under graph capture, tight serving loops, harnesses that
 * forbid hipMalloc).  The prefill K split's partial sums go to a static device array of
 * 64 MiB (one copy per GPU the library runs this on, held until the process ends; every
 * Llama-3-8B prefill shape fits).  A shape whose planned split needs more is refused with
 * OJX_ELAYOUT before any launch.  That refusal is a policy, not a limit of the kernels:
 * ojx_e8t_gemm_fwd would run such a shape with fewer splits, but a lower split count
 * changes the fp32 summation order, and this entry point promises the workspace entry
 * point's exact kernels, split and output.  All calls on one GPU share that GPU's array:
 * calls on one stream are ordered, calls that overlap on one GPU (other streams) race. */
int ojx_e8t_gemm_fwd_noalloc(const void* x, const uint8_t* packed, const uint16_t* scales,
                             const void* bias, void* y, int64_t M, int64_t N, int64_t K,
                             int64_t gs, int dtype, void* stream);

/* LoRA down-projection u[M, rank] = scaling * x[M, K] . A[K, rank] in fp32 (x and A in
 * dtype; 1 <= rank <= 64).  The first half of E8LatticeLinear's adapter term
 * scaling * ((x @ lora_A) @ lora_B) (ojasx2/math/lattice.py:839-842); the fused forwards
 * below (and grouped GEMV jobs with lora_r > 0) add u @ B in their output epilogue. */
int ojx_lora_down(const void* x, const void* lora_a, int64_t M, int64_t K, int64_t rank,
                  float scaling, int dtype, float* u, void* stream);

/* Fused forward with a LoRA adapter: y = x . Wdeq^T (+ bias) + scaling * (x @ A) @ B, the
 * adapter term added in fp32 before the one rounding to dtype.  Replaces the E8 op plus
 * the two matmuls and the add of E8LatticeLinear.forward (lattice.py:827-846; A [K, rank]
 * = lora_A, B [rank, N] = lora_B, both in dtype).  lora_u: caller-owned fp32 [M, rank]
 * scratch that receives u = scaling * (x @ A) (ojx_lora_down, launched first on the same
 * stream) -- except where the decode GEMV forms u inside its own launch (ternary, M <= 4 on
 * the staged-tile route with one 1024-k round per wave, rank 8, A 16-byte aligned): then
 * lora_u is not written.  Other arguments and the workspace as ojx_e8t_gemm_fwd; the e8 /
 * e8r variants take the 2-bit and 1-bit formats. */
int ojx_e8t_gemm_fwd_lora(const void* x, const uint8_t* packed, const uint16_t* scales,
                          const void* bias, const void* lora_a, const void* lora_b,
                          int64_t rank, float scaling, float* lora_u, void* y, int64_t M,
                          int64_t N, int64_t K, int64_t gs, int dtype, void* workspace,
                          size_t workspace_bytes, void* stream);
int ojx_e8_gemm_fwd_lora(const void* x, const uint8_t* packed, const uint16_t* scales,
                         const void* bias, const void* lora_a, const void* lora_b, int64_t rank,
                         float scaling, float* lora_u, void* y, int64_t M, int64_t N, int64_t K,
                         int64_t gs, int dtype, void* workspace, size_t workspace_bytes,
                         void* stream);
int ojx_e8r_gemm_fwd_lora(const void* x, const uint8_t* codes, const uint16_t* scales,
                          const void* bias, const void* lora_a, const void* lora_b,
                          int64_t rank, float scaling, float* lora_u, void* y, int64_t M,
                          int64_t N, int64_t K, int64_t gs, int dtype, void* workspace,
                          size_t workspace_bytes, void* stream);

/* Fused backward grad_x[M,K] = grad_y[M,N] . Wdeq[N,K], fp32 accumulation, in dtype.
 * Replaces fused_ternary_e8_gemm_bwd_dx (ojasx_math_bindings.cpp:479-533, schema :594);
 * called from _FusedE8GEMMFunction.backward (lattice.py:656-696).  Workspace as above. */
int ojx_e8t_gemm_bwd_dx(const void* grad_y, const uint8_t* packed, const uint16_t* scales,
                        void* grad_x, int64_t M, int64_t N, int64_t K, int64_t gs, int dtype,
                        void* workspace, size_t workspace_bytes, void* stream);

/* ---------------------------------------------------------------- 2-bit E8
 *
 * E8LatticePacker (2.0 bit/weight, ojasx2/math/lattice.py:209-279): four 2-bit codes per
 * byte (code j of a byte in bits [2j, 2j+2), the flat weight order), one fp16 scale per
 * flat group of gs weights; weight = (code - 1.5) * scale.
 *   packed  uint8 [padded / 4];  scales uint16 [padded / gs];  padded as above. */

/* Encoder, bit-exact with E8LatticePacker.pack (lattice.py:213-249).  gs a positive
 * multiple of 8 (the packer's ValueError, :220-221, is OJX_ELAYOUT here). */
int ojx_e8_encode(const void* w, int w_dtype, int64_t numel, int64_t gs, uint8_t* packed,
                  uint16_t* scales, void* stream);

/* Decoder, bit-exact with E8LatticePacker.unpack (lattice.py:252-279): out[i] =
 * (code - 1.5) * scales.to(dtype), the product rounded once to dtype.  gs a positive
 * multiple of 8. */
int ojx_e8_decode(const uint8_t* packed, const uint16_t* scales, int64_t numel, int64_t gs,
                  int out_dtype, void* out, void* stream);

/* Fused forward and backward dX over 2-bit weights, with the decoder's weight rule and
 * fp32 accumulation.  Replace fused_e8_gemm_fwd / fused_e8_gemm_bwd_dx
 * (ojasx_math_bindings.cpp:274-404, schemas :591-592) and the 2-bit portable path of
 * _FusedE8GEMMFunction (lattice.py:610-640, 684-717).  gs a positive multiple of 4 (the
 * native op's rule, bindings.cpp:285).  Any M, N, K (flat layout).  Workspace as for
 * ojx_e8t_gemm_fwd (fmt OJX_FMT_E8). */
int ojx_e8_gemm_fwd(const void* x, const uint8_t* packed, const uint16_t* scales,
                    const void* bias, void* y, int64_t M, int64_t N, int64_t K, int64_t gs,
                    int dtype, void* workspace, size_t workspace_bytes, void* stream);
int ojx_e8_gemm_bwd_dx(const void* grad_y, const uint8_t* packed, const uint16_t* scales,
                       void* grad_x, int64_t M, int64_t N, int64_t K, int64_t gs, int dtype,
                       void* workspace, size_t workspace_bytes, void* stream);

/* ---------------------------------------------------------------- 1-bit Root E8
 *
 * RootE8LatticePacker (1.0 bit/weight, ojasx2/math/lattice.py:426-533): one code byte per
 * flat 8-vector (an index into the reference's 256-entry table, :436-456), one fp16 scale
 * per flat group of gs weights; weight = table[code][k] * scale.
 *   codes  uint8 [padded / 8];  scales uint16 [padded / gs];  padded as above. */

/* Encoder, bit-exact with RootE8LatticePacker.pack (lattice.py:473-509): codes by the
 * argmax of v . u/|u| over the table rows (torch's CPU matmul order, first maximum), MMSE
 * scales sum(w q) / sum(q q) in torch's CPU sum order.  gs a positive multiple of 8 (the
 * packer coerces other values to 8, :485-486; that coercion is the caller's). */
int ojx_e8r_encode(const void* w, int w_dtype, int64_t numel, int64_t gs, uint8_t* codes,
                   uint16_t* scales, void* stream);

/* Decoder, bit-exact with RootE8LatticePacker.unpack (lattice.py:519-533): out[i] =
 * table[code][i % 8] * scales.to(dtype), rounded to dtype.  gs a positive multiple of 8. */
int ojx_e8r_decode(const uint8_t* codes, const uint16_t* scales, int64_t numel, int64_t gs,
                   int out_dtype, void* out, void* stream);

/* Fused forward and backward dX over 1-bit weights with the decoder's weight rule and
 * fp32 accumulation.  Replace the 1-bit portable path of _FusedE8GEMMFunction (unpack +
 * F.linear, lattice.py:610-640; backward :684-717).  gs a positive multiple of 8.  Any
 * M, N, K (flat layout).  Workspace as for ojx_e8t_gemm_fwd (fmt OJX_FMT_ROOT). */
int ojx_e8r_gemm_fwd(const void* x, const uint8_t* codes, const uint16_t* scales,
                     const void* bias, void* y, int64_t M, int64_t N, int64_t K, int64_t gs,
                     int dtype, void* workspace, size_t workspace_bytes, void* stream);
int ojx_e8r_gemm_bwd_dx(const void* grad_y, const uint8_t* codes, const uint16_t* scales,
                        void* grad_x, int64_t M, int64_t N, int64_t K, int64_t gs, int dtype,
                        void* workspace, size_t workspace_bytes, void* stream);

/* ---------------------------------------------------------------- Hadamard rotation
 *
 * fwht_block32 (ojasx2/math/lattice.py:91-102): the normalised 32-point Walsh-Hadamard
 * transform of each of the numel / 32 contiguous 32-element blocks of x into y (y == x is
 * allowed), with the reference's rounded operations (butterflies at distance 1, 2, 4, 8, 16,
 * each rounded to dtype; one multiply by 0.1767766952966369 in the compute type), so the
 * result is bit-identical to the torch evaluation.  The fused linear applies it to x before
 * the E8 op and to grad_x after the backward when use_hadamard is set (lattice.py:564-565,
 * 669-679, 713-714).  dtype: OJX_F32, OJX_F16, OJX_BF16 or OJX_F64; numel a multiple of 32;
 * x and y 16-byte aligned. */
int ojx_fwht32(const void* x, int dtype, int64_t numel, void* y, void* stream);

/* ---------------------------------------------------------------- QAT helpers
 *
 * Conway-Sloane nearest point of the E8 lattice for nvec contiguous 8-vectors, as
 * conway_sloane_e8_project's torch path computes it (ojasx2/math/lattice.py:162-203;
 * the reference's native CPU kernel, ojasx_math_core.hpp:385-425, rounds halves away from
 * zero instead).  x and out are fp32 (f64 = 0) or fp64 (f64 = 1). */
int ojx_e8_cs_project(const void* x, int f64, int64_t nvec, void* out, void* stream);

/* Forward of the QAT straight-through quantizer _E8STEFunction (lattice.py:853-865) on fp32
 * weights: per flat 8-vector (zero padded) s = torch.norm/sqrt(8) + 1e-8, out =
 * project(w / s) * s. */
int ojx_e8_ste_quantize(const float* w, int64_t numel, float* out, void* stream);

/* The projection for x and out in `dtype`: OJX_F32 or OJX_F64 as above, OJX_F16 or OJX_BF16
 * as the reference's torch expressions evaluate on such a tensor (lattice.py:180-203 in the
 * tensor's dtype): every elementwise op rounded to the dtype, sums over the 8 coordinates
 * added in fp32 and rounded once (the parity test reads that rounded sum). */
int ojx_e8_cs_project_dt(const void* x, int dtype, int64_t nvec, void* out, void* stream);

/* The STE forward for w and out in `dtype` (OJX_F32, OJX_F16 or OJX_BF16), every op of
 * lattice.py:855-865 rounded to the dtype: norm, / sqrt(8), + 1e-8 (an fp16 zero 8-vector
 * gets s = 0 and NaN outputs, as the reference does), w / s, the projection, * s. */
int ojx_e8_ste_quantize_dt(const void* w, int dtype, int64_t numel, void* out, void* stream);

/* ---------------------------------------------------------------- grouped decode GEMV
 *
 * One launch runs the decode GEMV (batch M <= 16) of several independent linears: a
 * decoder layer's q/k/v (or gate/up) projections sharing one x and writing one
 * concatenated output, or any table of linears (e.g. a whole layer stack).  This has no
 * single counterpart in the reference, whose decode path runs one unpack + GEMM per
 * linear (_FusedE8GEMMFunction.forward, lattice.py:610-624); the per-linear semantics of
 * each job are exactly those of ojx_e8t_gemm_fwd.
 *
 * Requirements per job: K % 256 == 0, group size 32, dtype F16 or BF16, 1 <= M <= 16,
 * x 16-byte aligned, packed and scales 4-byte aligned, y_ld >= y_col + N. */
typedef struct ojx_e8t_gemv_job {
    const void* x;          /* [M, K] activations; NULL = the launch's x          */
    const uint8_t* packed;  /* [N*K*3/16] codes of W[N, K]                        */
    const uint16_t* scales; /* [N*K/32] fp16 scale bits                           */
    const void* bias;       /* [N] in dtype, or NULL                              */
    void* y;                /* output base; NULL = the launch's y                  */
    int64_t N, K;
    int64_t y_col;          /* y[m, y_col + n] receives output n of row m          */
    int64_t y_ld;           /* row stride of y in elements (0 means N)             */
    int64_t wg_begin;       /* written by ojx_e8t_gemv_grouped_plan                */
    /* LoRA adapter (lora_r in 1..64; 0 = none), E8LatticeLinear.forward's
     * scaling * ((x @ A) @ B) (lattice.py:839-842): ojx_e8t_gemv_grouped first writes
     * u = lora_scaling * (x @ A) into the caller's fp32 scratch lora_u [M, lora_r] (row
     * stride lora_ldu, 0 = lora_r; adapters on the same x share one launch), then the
     * GEMV adds u @ B before the output is rounded.  A [K, lora_r], B [lora_r, N] in
     * dtype.  A launch on the staged-tile kernel with one round per wave and one row tile
     * per workgroup (small grouped launches, M <= 4) forms u itself when every adapter has
     * rank 8 and a 16-byte aligned A: one launch, lora_u not written. */
    float* lora_u;
    const void* lora_b;
    int64_t lora_r;
    int64_t lora_ldu;
    const void* lora_a;
    float lora_scaling;
    int32_t reserved;       /* 0 */
} ojx_e8t_gemv_job;

/* Validates `jobs` (host array) for batch M and dtype, fills each wg_begin (and y_ld
 * when 0) and returns the launch grid in *grid.  A planned array may be copied to
 * device memory once and reused for every launch with the same M. */
int ojx_e8t_gemv_grouped_plan(ojx_e8t_gemv_job* jobs, int njobs, int64_t M, int dtype,
                              int64_t* grid);

/* Workgroups are issued in job order, and a job's workgroups run K / 1024 rounds each:
 * ordering the jobs by decreasing K keeps the longest workgroups from forming the launch's
 * tail (ojasx_amd.grouped.GroupedGemv does so). */

/* Launches a planned group.  `jobs` is the planned host array; `jobs_dev` is NULL (then
 * njobs <= 4 and the jobs travel in the kernel arguments) or a device copy of `jobs`.
 * `x` and `y` are the defaults for jobs whose x / y are NULL. */
int ojx_e8t_gemv_grouped(const ojx_e8t_gemv_job* jobs, const ojx_e8t_gemv_job* jobs_dev,
                         int njobs, const void* x, void* y, int64_t M, int dtype, void* stream);

/* The same for 2-bit E8 linears (E8LatticePacker, the reference's default bitrate,
 * lattice.py:210-279, 735, 906): `packed` is [N * K / 4] bytes, `scales` [N * K / gs] fp16,
 * every job with the one group size gs (8, 16, 32 or 64).  Requirements per job: K % 256 ==
 * 0, 1 <= M <= 16, packed / scales / x 16-byte aligned; adapters as above (their
 * down-projections run before the GEMV).  M <= 4 with every K a multiple of 1024 runs the
 * post-scaled 2-bit kernel, otherwise the B-operand kernel.  No counterpart in the
 * reference, which decodes each linear to a dense matrix (lattice.py:610-624). */
int ojx_e8_gemv_grouped_plan(ojx_e8t_gemv_job* jobs, int njobs, int64_t M, int64_t gs,
                             int dtype, int64_t* grid);
int ojx_e8_gemv_grouped(const ojx_e8t_gemv_job* jobs, const ojx_e8t_gemv_job* jobs_dev,
                        int njobs, const void* x, void* y, int64_t M, int64_t gs, int dtype,
                        void* stream);

/* The same for 1-bit Root E8 linears (RootE8LatticePacker, lattice.py:426-533): `packed` is
 * [N * K / 8] bytes (one 8-bit code per 8 weights), `scales` [N * K / gs] fp16, gs 8, 16, 32
 * or 64; the B-operand kernel at every M.  No counterpart in the reference (its 1-bit
 * forward unpacks each linear, lattice.py:610-640). */
int ojx_e8r_gemv_grouped_plan(ojx_e8t_gemv_job* jobs, int njobs, int64_t M, int64_t gs,
                              int dtype, int64_t* grid);
int ojx_e8r_gemv_grouped(const ojx_e8t_gemv_job* jobs, const ojx_e8t_gemv_job* jobs_dev,
                         int njobs, const void* x, void* y, int64_t M, int64_t gs, int dtype,
                         void* stream);

#ifdef __cplusplus
}
#endif

#endif /* OJASX_E8T_H */
