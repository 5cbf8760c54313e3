/*
 * e8t_oracle.c -- CPU restatement of the reference's ternary-E8 (1.5 bit/weight)
 * codec and of its dequantize-then-matmul forward.
 *
 * TEST INFRASTRUCTURE ONLY.  This file is the checker: only tests/, the smoke
 * check in __graft_entry__.py and bench.py's cpu_baseline leg load it.  The
 * product (the HIP library under ojasx-open-source-cuda_amd/) never links it.
 *
 * Every function follows the reference's Python (ojasx2/math/lattice.py) step by
 * step, at fp32 with no FMA contraction except where torch itself fuses (the
 * vectorised norm).  Build with -ffp-contract=off (see oracle/Makefile).
 *
 * Reference anchors:
 *   codebook            lattice.py:292-332   (rank = raw/2 closed form; checked
 *                                             against the reference's own C++ LUT,
 *                                             ojasx_math_core.hpp:549-573, via oracle/_ref)
 *   encoder             lattice.py:338-384
 *   decoder             lattice.py:386-419
 *   portable forward    lattice.py:610-624  (unpack + F.linear)
 *
 * The 2-bit E8 codec (E8LatticePacker, lattice.py:209-279) and its dequantize-then-
 * matmul follow in the section "2-bit E8" below (ojo_e8b_*).
 *
 * Pinning of each function (tests/test_oracle_*.py):
 *   ojo_f32_to_f16 / ojo_f32_to_bf16   vs numpy / torch conversions (library)
 *   ojo_e8t_group_scale                vs torch.norm(...)/math.sqrt(gs)+1e-8 (library)
 *   ojo_e8t_quantize8                  vs exhaustive nearest-point search over the 3,281
 *                                      codewords in exact arithmetic, plus hand-derived
 *                                      tie cases (tests/golden/known_answers.json)
 *   ojo_e8t_encode / _decode           byte layout closed form, the reference tests'
 *                                      invariants (size, cos > 0.7, row-wise == whole)
 *   ojo_e8t_gemm_f64                   vs the reference's C++ fused GEMV (oracle/_ref)
 *   ojo_e8b_quantize8                  vs exhaustive nearest-point search over the even-
 *                                      parity half-integer codewords for unclamped vectors,
 *                                      plus hand-derived clamp / tie cases
 *                                      (tests/golden/known_answers_e8b.json)
 *   ojo_e8b_encode / _decode           byte layout closed form, the reference tests'
 *                                      invariants, torch's own dtype products
 *   ojo_e8b_gemm_f64 / _bwd_f64        vs the reference's C++ 2-bit fused GEMM and
 *                                      backward (ojasx_math_core.hpp:440-534, oracle/_ref)
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

#ifdef _OPENMP
#include <omp.h>
#endif

#define OJO_API __attribute__((visibility("default")))

static const int32_t kPow3[8] = {1, 3, 9, 27, 81, 243, 729, 2187};

/* ------------------------------------------------------------------------- */
/* Number format conversions (IEEE binary16 and bfloat16, round-nearest-even) */
/* ------------------------------------------------------------------------- */

static inline uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

/* fp32 -> fp16, RNE, subnormals kept, overflow -> inf, NaN -> quiet NaN.
 * Same results as torch's Tensor.to(torch.float16) on CPU (pack, lattice.py:384). */
OJO_API uint16_t ojo_f32_to_f16(float f) {
    uint32_t x = f2u(f);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t ax = x & 0x7FFFFFFFu;
    if (ax >= 0x7F800000u) return (uint16_t)(sign | (ax > 0x7F800000u ? 0x7E00u : 0x7C00u));
    uint32_t e = ax >> 23;
    if (e < 113) { /* below 2^-14: half subnormal (or zero) */
        if (e == 0) return (uint16_t)sign; /* fp32 subnormal: far below half range */
        uint32_t mant = (ax & 0x7FFFFFu) | 0x800000u;
        uint32_t shift = 126 - e; /* value / 2^-24 = mant * 2^(e-126) */
        if (shift > 24) return (uint16_t)sign; /* < 2^-25 (or == with even result) */
        uint32_t q = mant >> shift;
        uint32_t rem = mant & ((1u << shift) - 1u);
        uint32_t half = 1u << (shift - 1);
        if (rem > half || (rem == half && (q & 1u))) q++;
        return (uint16_t)(sign | q);
    }
    uint32_t he = e - 112; /* rebias 127 -> 15 */
    uint32_t mant = ax & 0x7FFFFFu;
    uint32_t q = (he << 10) | (mant >> 13);
    uint32_t rem = mant & 0x1FFFu;
    if (rem > 0x1000u || (rem == 0x1000u && (q & 1u))) q++;
    if (q >= 0x7C00u) q = 0x7C00u; /* overflow to inf */
    return (uint16_t)(sign | q);
}

OJO_API float ojo_f16_to_f32(uint16_t h) {
    uint32_t sign = ((uint32_t)h & 0x8000u) << 16;
    uint32_t e = (h >> 10) & 0x1Fu;
    uint32_t m = h & 0x3FFu;
    if (e == 0x1F) return u2f(sign | 0x7F800000u | (m << 13));
    if (e == 0) {
        /* subnormal: m * 2^-24, exact in fp32 */
        float v = (float)m * 5.9604644775390625e-08f;
        return sign ? -v : v;
    }
    return u2f(sign | ((e + 112) << 23) | (m << 13));
}

/* fp32 -> bf16, RNE, NaN -> 0x7FC0 (c10::BFloat16 round_to_nearest_even). */
OJO_API uint16_t ojo_f32_to_bf16(float f) {
    uint32_t u = f2u(f);
    if ((u & 0x7FFFFFFFu) > 0x7F800000u) return 0x7FC0u;
    u += 0x7FFFu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

OJO_API float ojo_bf16_to_f32(uint16_t b) { return u2f((uint32_t)b << 16); }

/* ------------------------------------------------------------------------- */
/* Codebook: D8 cap {-1,0,1}^8 with even coordinate sum, 3,281 points.         */
/* lattice.py:309-318 enumerates raw = sum (q_i+1) 3^i in increasing order and  */
/* keeps even-digit-sum entries; since 3^i is odd, digit-sum parity == raw      */
/* parity, so rank = raw / 2 and raw = 2 * rank.                               */
/* ------------------------------------------------------------------------- */

OJO_API void ojo_e8t_codeword(int32_t code, int8_t coords[8]) {
    int32_t raw = 2 * code;
    for (int i = 0; i < 8; ++i) {
        coords[i] = (int8_t)(raw % 3 - 1);
        raw /= 3;
    }
}

/* ------------------------------------------------------------------------- */
/* Encoder                                                                     */
/* ------------------------------------------------------------------------- */

/* Scale of one flat group (lattice.py:355-356):
 *   s = torch.norm(w_g) / math.sqrt(gs) + 1e-8       (fp32 throughout)
 * torch's CPU norm over the last dim keeps 8 fp32 FMA lanes, lane j summing
 * w[j], w[j+8], ... in order, then adds the 8 lanes left to right, then takes a
 * correctly rounded sqrt.  The python scalar sqrt(gs) is rounded to fp32 before
 * the (true) division. */
OJO_API float ojo_e8t_group_scale(const float* w, int64_t gs) {
    float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    for (int64_t k = 0; k < gs; k += 8)
        for (int j = 0; j < 8; ++j) acc[j] = fmaf(w[k + j], w[k + j], acc[j]);
    float sum = acc[0];
    for (int j = 1; j < 8; ++j) sum = sum + acc[j];
    float nrm = sqrtf(sum);
    float root = (float)sqrt((double)gs);
    float s = nrm / root;
    return s + 1e-8f;
}

/* Nearest point of one 8-vector v (already divided by the scale), following
 * lattice.py:358-373 exactly:
 *   q   = clamp(round_half_even(v), -1, 1)
 *   alt = (q == 0) ? (v >= 0 ? +1 : -1) : 0
 *   pen = (alt - v)^2 - (q - v)^2            (three separately rounded ops)
 *   if sum(q) is odd: q[first argmin pen] = alt[...]
 *   code = (sum (q_i + 1) 3^i) / 2
 * Returns the 12-bit code; writes the chosen coordinates to q_out if non-null. */
OJO_API int32_t ojo_e8t_quantize8(const float v[8], int8_t q_out[8]) {
    float q[8], alt[8], pen[8];
    int sum = 0;
    for (int i = 0; i < 8; ++i) {
        float r = rintf(v[i]); /* default rounding mode: nearest-even */
        if (r < -1.0f) r = -1.0f;
        if (r > 1.0f) r = 1.0f;
        q[i] = r;
        sum += (int)r;
    }
    for (int i = 0; i < 8; ++i) {
        alt[i] = (q[i] == 0.0f) ? (v[i] >= 0.0f ? 1.0f : -1.0f) : 0.0f;
        float a = alt[i] - v[i];
        float b = q[i] - v[i];
        float a2 = a * a;
        float b2 = b * b;
        pen[i] = a2 - b2;
    }
    if (sum & 1) {
        int best = 0;
        for (int i = 1; i < 8; ++i)
            if (pen[i] < pen[best]) best = i;
        q[best] = alt[best];
    }
    int32_t raw = 0;
    for (int i = 0; i < 8; ++i) {
        int d = (int)q[i] + 1;
        raw += d * kPow3[i];
        if (q_out) q_out[i] = (int8_t)(d - 1);
    }
    return raw >> 1;
}

static inline void put_pair(uint8_t* dst, int32_t c0, int32_t c1) {
    /* lattice.py:379-383: two 12-bit codes, little-endian bit stream */
    dst[0] = (uint8_t)(c0 & 0xFF);
    dst[1] = (uint8_t)(((c0 >> 8) & 0x0F) | ((c1 & 0x0F) << 4));
    dst[2] = (uint8_t)((c1 >> 4) & 0xFF);
}

/* Encode one flat group of gs fp32 weights. */
static void encode_group(const float* w, int64_t gs, uint8_t* packed, uint16_t* scale16,
                         float* scale32) {
    float s = ojo_e8t_group_scale(w, gs);
    int32_t codes[2];
    for (int64_t t = 0; t < gs / 8; ++t) {
        float v[8];
        for (int i = 0; i < 8; ++i) v[i] = w[8 * t + i] / s;
        codes[t & 1] = ojo_e8t_quantize8(v, 0);
        if (t & 1) put_pair(packed + 3 * (t >> 1), codes[0], codes[1]);
    }
    *scale16 = ojo_f32_to_f16(s);
    if (scale32) *scale32 = s;
}

/* Padded element count used by the reference (flat zero padding to a multiple of gs). */
OJO_API int64_t ojo_e8t_padded(int64_t numel, int64_t gs) {
    return numel + ((gs - numel % gs) % gs);
}

/* Effective group size: the reference silently coerces gs to 16 when it is not a
 * positive multiple of 16 (lattice.py:346-347). */
OJO_API int64_t ojo_e8t_effective_gs(int64_t gs) {
    return (gs <= 0 || gs % 16 != 0) ? 16 : gs;
}

/* TernaryE8LatticePacker.pack on a flat fp32 array of numel values.
 * packed: padded*3/16 bytes; scales: padded/gs fp16 bit patterns;
 * scales32 (optional): the fp32 scales the codes were computed with. */
OJO_API void ojo_e8t_encode(const float* w, int64_t numel, int64_t gs, uint8_t* packed,
                            uint16_t* scales, float* scales32, int nthreads) {
    gs = ojo_e8t_effective_gs(gs);
    int64_t padded = ojo_e8t_padded(numel, gs);
    int64_t ngroups = padded / gs;
    int64_t full = numel / gs;
#ifdef _OPENMP
    if (nthreads <= 0) nthreads = omp_get_max_threads();
#pragma omp parallel for schedule(static) num_threads(nthreads)
#endif
    for (int64_t g = 0; g < full; ++g)
        encode_group(w + g * gs, gs, packed + g * gs * 3 / 16, scales + g,
                     scales32 ? scales32 + g : 0);
    (void)nthreads;
    if (full < ngroups) { /* tail group, zero padded (F.pad) */
        float tmp[4096];
        float* buf = tmp;
        if (gs > 4096) return; /* not reachable from the tests */
        int64_t rem = numel - full * gs;
        for (int64_t i = 0; i < gs; ++i) buf[i] = i < rem ? w[full * gs + i] : 0.0f;
        encode_group(buf, gs, packed + full * gs * 3 / 16, scales + full,
                     scales32 ? scales32 + full : 0);
    }
}

/* ------------------------------------------------------------------------- */
/* Decoder                                                                     */
/* ------------------------------------------------------------------------- */

static inline int32_t get_code(const uint8_t* packed, int64_t t) {
    const uint8_t* b = packed + 3 * (t >> 1);
    if ((t & 1) == 0) return (int32_t)b[0] | ((int32_t)(b[1] & 0x0F) << 8);
    return (int32_t)(b[1] >> 4) | ((int32_t)b[2] << 4);
}

/* Decoded weight value as the reference's unpack produces it for out dtype
 * (lattice.py:412-419): coords.to(dtype) * scales.to(dtype).
 *   dtype 0 (fp32): coord * float(s16)            (exact)
 *   dtype 1 (fp16): coord * s16                   (exact)
 *   dtype 2 (bf16): coord * bf16_rne(float(s16))  (exact after the scale cast) */
static inline float deq_value(int coord, uint16_t s16, int dtype) {
    float s = ojo_f16_to_f32(s16);
    if (dtype == 2) s = ojo_bf16_to_f32(ojo_f32_to_bf16(s));
    return (float)coord * s;
}

/* Unpack into numel (unpadded prefix) values.  out_dtype: 0 f32, 1 f16 bits,
 * 2 bf16 bits.  gs is the group size (the reference infers padded/numel(scales)). */
OJO_API void ojo_e8t_decode(const uint8_t* packed, const uint16_t* scales, int64_t numel,
                            int64_t gs, int out_dtype, void* out) {
    int64_t ncodes = (numel + 7) / 8;
#ifdef _OPENMP
#pragma omp parallel for schedule(static)
#endif
    for (int64_t t = 0; t < ncodes; ++t) {
        int32_t raw = 2 * get_code(packed, t);
        uint16_t s16 = scales[(8 * t) / gs];
        for (int i = 0; i < 8; ++i) {
            int coord = raw % 3 - 1;
            raw /= 3;
            int64_t idx = 8 * t + i;
            if (idx >= numel) break;
            float v = deq_value(coord, s16, out_dtype);
            if (out_dtype == 0) ((float*)out)[idx] = v;
            else if (out_dtype == 1) ((uint16_t*)out)[idx] = ojo_f32_to_f16(v);
            else ((uint16_t*)out)[idx] = ojo_f32_to_bf16(v);
        }
    }
}

/* ------------------------------------------------------------------------- */
/* Dequantize-then-matmul reference (fp64 accumulation)                       */
/* ------------------------------------------------------------------------- */

/* y[m,n] = sum_k x[m,k] * Wdeq[n,k] + bias[n], accumulated in fp64, with Wdeq
 * decoded exactly as the reference's portable path decodes for dtype w_dtype
 * (lattice.py:618-623).  x, bias fp32 (the caller widens bf16/fp16 inputs
 * exactly).  Requires the row layout K % gs == 0 (one row = whole groups). */
OJO_API void ojo_e8t_gemm_f64(const float* x, const uint8_t* packed, const uint16_t* scales,
                              const float* bias, double* y, int64_t M, int64_t N, int64_t K,
                              int64_t gs, int w_dtype) {
#ifdef _OPENMP
#pragma omp parallel for schedule(static)
#endif
    for (int64_t n = 0; n < N; ++n) {
        double wrow_buf[16384];
        double* wrow = wrow_buf;
        if (K > 16384) continue; /* not reachable from the tests */
        for (int64_t t = 0; t < K / 8; ++t) {
            int64_t tt = n * (K / 8) + t;
            int32_t raw = 2 * get_code(packed, tt);
            uint16_t s16 = scales[(8 * tt) / gs];
            for (int i = 0; i < 8; ++i) {
                int coord = raw % 3 - 1;
                raw /= 3;
                wrow[8 * t + i] = (double)deq_value(coord, s16, w_dtype);
            }
        }
        for (int64_t m = 0; m < M; ++m) {
            double acc = bias ? (double)bias[n] : 0.0;
            const float* xr = x + m * K;
            for (int64_t k = 0; k < K; ++k) acc += (double)xr[k] * wrow[k];
            y[m * N + n] = acc;
        }
    }
}

/* grad_x[m,k] = sum_n gy[m,n] * Wdeq[n,k] (fp64), the reference's backward
 * (lattice.py:686-696). */
OJO_API void ojo_e8t_gemm_bwd_f64(const float* gy, const uint8_t* packed, const uint16_t* scales,
                                  double* gx, int64_t M, int64_t N, int64_t K, int64_t gs,
                                  int w_dtype) {
    memset(gx, 0, sizeof(double) * (size_t)(M * K));
    for (int64_t n = 0; n < N; ++n) {
        for (int64_t t = 0; t < K / 8; ++t) {
            int64_t tt = n * (K / 8) + t;
            int32_t raw = 2 * get_code(packed, tt);
            uint16_t s16 = scales[(8 * tt) / gs];
            for (int i = 0; i < 8; ++i) {
                int coord = raw % 3 - 1;
                raw /= 3;
                double wv = (double)deq_value(coord, s16, w_dtype);
                if (wv == 0.0) continue;
                for (int64_t m = 0; m < M; ++m) gx[m * K + 8 * t + i] += (double)gy[m * N + n] * wv;
            }
        }
    }
}

/* ------------------------------------------------------------------------- */
/* Array helpers for the Python test wrapper                                  */
/* ------------------------------------------------------------------------- */

OJO_API void ojo_f32_to_f16_array(const float* in, uint16_t* out, int64_t n) {
    for (int64_t i = 0; i < n; ++i) out[i] = ojo_f32_to_f16(in[i]);
}
OJO_API void ojo_f32_to_bf16_array(const float* in, uint16_t* out, int64_t n) {
    for (int64_t i = 0; i < n; ++i) out[i] = ojo_f32_to_bf16(in[i]);
}
OJO_API void ojo_e8t_group_scale_array(const float* w, int64_t ngroups, int64_t gs, float* out) {
    for (int64_t g = 0; g < ngroups; ++g) out[g] = ojo_e8t_group_scale(w + g * gs, gs);
}
OJO_API void ojo_e8t_quantize8_array(const float* v, int64_t nvec, int32_t* codes) {
    for (int64_t t = 0; t < nvec; ++t) codes[t] = ojo_e8t_quantize8(v + 8 * t, 0);
}

/* ------------------------------------------------------------------------- */
/* 2-bit E8 (E8LatticePacker, lattice.py:209-279)                             */
/* ------------------------------------------------------------------------- */

/* Group size rule of E8LatticePacker.pack (lattice.py:220-221): a positive multiple of 8,
 * otherwise ValueError (the caller checks; -1 here). */
OJO_API int64_t ojo_e8b_check_gs(int64_t gs) { return (gs <= 0 || gs % 8 != 0) ? -1 : gs; }

/* One 8-vector v (already divided by the scale), lattice.py:229-238 step by step:
 *   xs  = v - 0.5
 *   f2  = clamp(round_half_even(xs), -2, 1)
 *   alt = (xs >= f2) ? clamp(f2 + 1, -2, 1) : clamp(f2 - 1, -2, 1)
 *   pen = (alt - xs)^2 - (f2 - xs)^2          (five separately rounded fp32 ops)
 *   if sum(f2) is odd: f2[first argmin pen] = alt[...]
 *   code_i = f2_i + 2                          (= clamp(round(f2 + 0.5 + 1.5), 0, 3))
 * A coordinate clamped at -2 or 1 has alt == f2 and pen == 0: when it is the first
 * minimum, the "flip" changes nothing and the vector keeps an odd sum, as the
 * reference's does.  Writes the 8 codes (0..3) to codes[]. */
OJO_API void ojo_e8b_quantize8(const float v[8], uint8_t codes[8]) {
    float xs[8], f2[8], alt[8], pen[8];
    float sum = 0.0f;
    for (int i = 0; i < 8; ++i) {
        xs[i] = v[i] - 0.5f;
        float r = rintf(xs[i]);
        if (r < -2.0f) r = -2.0f;
        if (r > 1.0f) r = 1.0f;
        f2[i] = r;
        sum += r; /* small integers: exact */
    }
    for (int i = 0; i < 8; ++i) {
        float up = f2[i] + 1.0f, dn = f2[i] - 1.0f;
        if (up > 1.0f) up = 1.0f;
        if (dn < -2.0f) dn = -2.0f;
        alt[i] = (xs[i] >= f2[i]) ? up : dn;
        float a = alt[i] - xs[i];
        float b = f2[i] - xs[i];
        float a2 = a * a;
        float b2 = b * b;
        pen[i] = a2 - b2;
    }
    if (((int)sum) & 1) {
        int best = 0;
        for (int i = 1; i < 8; ++i)
            if (pen[i] < pen[best]) best = i;
        f2[best] = alt[best];
    }
    for (int i = 0; i < 8; ++i) codes[i] = (uint8_t)((int)f2[i] + 2);
}

/* Encode one flat group of gs fp32 weights: scale as the ternary packer's
 * (lattice.py:227 is the same expression), codes 4 per byte, code j of a byte in
 * bits [2j, 2j+2) (lattice.py:242-247). */
static void e8b_encode_group(const float* w, int64_t gs, uint8_t* packed, uint16_t* scale16,
                             float* scale32) {
    float s = ojo_e8t_group_scale(w, gs);
    for (int64_t t = 0; t < gs / 8; ++t) {
        float v[8];
        uint8_t c[8];
        for (int i = 0; i < 8; ++i) v[i] = w[8 * t + i] / s;
        ojo_e8b_quantize8(v, c);
        packed[2 * t] = (uint8_t)(c[0] | (c[1] << 2) | (c[2] << 4) | (c[3] << 6));
        packed[2 * t + 1] = (uint8_t)(c[4] | (c[5] << 2) | (c[6] << 4) | (c[7] << 6));
    }
    *scale16 = ojo_f32_to_f16(s);
    if (scale32) *scale32 = s;
}

/* E8LatticePacker.pack on a flat fp32 array of numel values (gs a positive multiple
 * of 8).  packed: padded/4 bytes; scales: padded/gs fp16 bits; scales32 optional. */
OJO_API void ojo_e8b_encode(const float* w, int64_t numel, int64_t gs, uint8_t* packed,
                            uint16_t* scales, float* scales32, int nthreads) {
    int64_t padded = ojo_e8t_padded(numel, gs);
    int64_t ngroups = padded / gs;
    int64_t full = numel / gs;
#ifdef _OPENMP
    if (nthreads <= 0) nthreads = omp_get_max_threads();
#pragma omp parallel for schedule(static) num_threads(nthreads)
#endif
    for (int64_t g = 0; g < full; ++g)
        e8b_encode_group(w + g * gs, gs, packed + g * gs / 4, scales + g,
                         scales32 ? scales32 + g : 0);
    (void)nthreads;
    if (full < ngroups) { /* tail group, zero padded (F.pad, lattice.py:223-225) */
        float buf[4096];
        if (gs > 4096) return; /* not reachable from the tests */
        int64_t rem = numel - full * gs;
        for (int64_t i = 0; i < gs; ++i) buf[i] = i < rem ? w[full * gs + i] : 0.0f;
        e8b_encode_group(buf, gs, packed + full * gs / 4, scales + full,
                         scales32 ? scales32 + full : 0);
    }
}

/* Decoded weight as E8LatticePacker.unpack produces it for out dtype
 * (lattice.py:274-276): (codes.to(dtype) - 1.5) * scales.to(dtype), the product
 * rounded to dtype (torch computes it in fp32 and rounds once).
 *   dtype 0 (fp32): (c - 1.5) * float(s16)                exact
 *   dtype 1 (fp16): fp16_rne((c - 1.5) * float(s16))
 *   dtype 2 (bf16): bf16_rne((c - 1.5) * bf16_rne(float(s16))) */
static inline float e8b_deq_value(int code, uint16_t s16, int dtype) {
    float s = ojo_f16_to_f32(s16);
    if (dtype == 2) s = ojo_bf16_to_f32(ojo_f32_to_bf16(s));
    float p = ((float)code - 1.5f) * s; /* exact in fp32 */
    if (dtype == 1) return ojo_f16_to_f32(ojo_f32_to_f16(p));
    if (dtype == 2) return ojo_bf16_to_f32(ojo_f32_to_bf16(p));
    return p;
}

static inline int e8b_code(const uint8_t* packed, int64_t f) {
    return (packed[f >> 2] >> (2 * (f & 3))) & 3;
}

/* Unpack into numel values; gs = padded / numel(scales) as the reference infers it
 * (lattice.py:264-266).  out_dtype: 0 f32, 1 f16 bits, 2 bf16 bits. */
OJO_API void ojo_e8b_decode(const uint8_t* packed, const uint16_t* scales, int64_t numel,
                            int64_t gs, int out_dtype, void* out) {
#ifdef _OPENMP
#pragma omp parallel for schedule(static)
#endif
    for (int64_t f = 0; f < numel; ++f) {
        float v = e8b_deq_value(e8b_code(packed, f), scales[f / gs], out_dtype);
        if (out_dtype == 0) ((float*)out)[f] = v;
        else if (out_dtype == 1) ((uint16_t*)out)[f] = ojo_f32_to_f16(v);
        else ((uint16_t*)out)[f] = ojo_f32_to_bf16(v);
    }
}

/* y = x . Wdeq^T + bias in fp64, Wdeq by the dtype rule above (the portable path,
 * lattice.py:618-623).  Flat layout: element (n, k) is flat index n*K + k. */
OJO_API void ojo_e8b_gemm_f64(const float* x, const uint8_t* packed, const uint16_t* scales,
                              const float* bias, double* y, int64_t M, int64_t N, int64_t K,
                              int64_t gs, int w_dtype) {
#ifdef _OPENMP
#pragma omp parallel for schedule(static)
#endif
    for (int64_t n = 0; n < N; ++n) {
        double wrow_buf[16384];
        double* wrow = wrow_buf;
        if (K > 16384) continue; /* not reachable from the tests */
        for (int64_t k = 0; k < K; ++k) {
            int64_t f = n * K + k;
            wrow[k] = (double)e8b_deq_value(e8b_code(packed, f), scales[f / gs], w_dtype);
        }
        for (int64_t m = 0; m < M; ++m) {
            double acc = bias ? (double)bias[n] : 0.0;
            const float* xr = x + m * K;
            for (int64_t k = 0; k < K; ++k) acc += (double)xr[k] * wrow[k];
            y[m * N + n] = acc;
        }
    }
}

/* grad_x = gy . Wdeq in fp64 (lattice.py:686-696 with the 2-bit unpack). */
OJO_API void ojo_e8b_gemm_bwd_f64(const float* gy, const uint8_t* packed, const uint16_t* scales,
                                  double* gx, int64_t M, int64_t N, int64_t K, int64_t gs,
                                  int w_dtype) {
    memset(gx, 0, sizeof(double) * (size_t)(M * K));
    for (int64_t n = 0; n < N; ++n)
        for (int64_t k = 0; k < K; ++k) {
            int64_t f = n * K + k;
            double wv = (double)e8b_deq_value(e8b_code(packed, f), scales[f / gs], w_dtype);
            for (int64_t m = 0; m < M; ++m) gx[m * K + k] += (double)gy[m * N + n] * wv;
        }
}

OJO_API void ojo_e8b_quantize8_array(const float* v, int64_t nvec, uint8_t* codes) {
    for (int64_t t = 0; t < nvec; ++t) ojo_e8b_quantize8(v + 8 * t, codes + 8 * t);
}

/* ------------------------------------------------------------------------- */
/* 1-bit Root E8 (RootE8LatticePacker, lattice.py:426-533)                      */
/* ------------------------------------------------------------------------- */

/* The 256-entry table of lattice.py:436-456, scaled by 2 as the reference scales it:
 *   0..111   (+-2 at i, +-2 at j), i < j, loops i, j, s1 in (-1, +1), s2 in (-1, +1)
 *   112..239 (+-1)^8 with an even number of -1, in itertools.product order over
 *            (-0.5, +0.5) (first coordinate slowest), scaled
 *   240..255 (+-2 at i), loops i, s in (-1, +1) */
OJO_API void ojo_e8r_lut(float out[256 * 8]) {
    int e = 0;
    memset(out, 0, 256 * 8 * sizeof(float));
    for (int i = 0; i < 8; ++i)
        for (int j = i + 1; j < 8; ++j)
            for (int a = 0; a < 2; ++a)
                for (int b = 0; b < 2; ++b) {
                    out[8 * e + i] = a ? 2.0f : -2.0f;
                    out[8 * e + j] = b ? 2.0f : -2.0f;
                    ++e;
                }
    for (int p = 0; p < 256; ++p) {
        int neg = 0;
        for (int k = 0; k < 8; ++k) neg += !((p >> (7 - k)) & 1);
        if (neg & 1) continue;
        for (int k = 0; k < 8; ++k) out[8 * e + k] = ((p >> (7 - k)) & 1) ? 1.0f : -1.0f;
        ++e;
    }
    for (int i = 0; i < 8; ++i)
        for (int s = 0; s < 2; ++s) {
            out[8 * e + i] = s ? 2.0f : -2.0f;
            ++e;
        }
}

/* Code of one 8-vector v (already divided by the group's initial scale), as
 * argmax(v . normalize(lut)^T) (lattice.py:497-500): each dot product is the
 * sequential FMA chain acc = fmaf(v[k], u[k], acc) from acc = +0 over k = 0..7 (the
 * order of torch's CPU matmul for these shapes, checked against torch), u the table
 * row divided by its norm in fp32; the first maximal index wins (torch.argmax). */
OJO_API int32_t ojo_e8r_quantize8(const float v[8]) {
    static float unorm[256 * 8];
    static int ready = 0;
    if (!ready) { /* not thread-safe on first use: callers warm it up (ojo_e8r_prepare) */
        float lut[256 * 8];
        ojo_e8r_lut(lut);
        for (int e = 0; e < 256; ++e) {
            float ss = 0.0f;
            for (int k = 0; k < 8; ++k) ss = ss + lut[8 * e + k] * lut[8 * e + k];
            float n = sqrtf(ss);
            if (n < 1e-12f) n = 1e-12f;
            for (int k = 0; k < 8; ++k) unorm[8 * e + k] = lut[8 * e + k] / n;
        }
        ready = 1;
    }
    int best = 0;
    float best_dot = 0.0f;
    for (int e = 0; e < 256; ++e) {
        float acc = 0.0f;
        for (int k = 0; k < 8; ++k) acc = fmaf(v[k], unorm[8 * e + k], acc);
        if (e == 0 || acc > best_dot) {
            best = e;
            best_dot = acc;
        }
    }
    return best;
}

OJO_API void ojo_e8r_prepare(void) {
    float v[8] = {0};
    (void)ojo_e8r_quantize8(v);
}

/* Sum over a group of gs values in the order of torch's CPU sum along a contiguous last
 * dim (checked against torch for every multiple of 8 up to 256): four 8-lane
 * accumulators take the 8-blocks of each 32-block in turn, 8-blocks after the last full
 * 32-block go to the first accumulator, the four accumulators are added in order and
 * then their 8 lanes left to right. */
static float torch_row_sum(const float* x, int64_t n) {
    float acc[4][8];
    memset(acc, 0, sizeof(acc));
    int64_t nch = n / 8, main = (nch / 4) * 4;
    for (int64_t c = 0; c < nch; ++c) {
        int a = c < main ? (int)(c % 4) : 0;
        for (int j = 0; j < 8; ++j) acc[a][j] = acc[a][j] + x[8 * c + j];
    }
    float lane[8];
    for (int j = 0; j < 8; ++j) lane[j] = ((acc[0][j] + acc[1][j]) + acc[2][j]) + acc[3][j];
    float s = lane[0];
    for (int j = 1; j < 8; ++j) s = s + lane[j];
    return s;
}

OJO_API float ojo_e8r_row_sum(const float* x, int64_t n) { return torch_row_sum(x, n); }

/* One flat group (lattice.py:486-509): initial scale as the other packers', codes by
 * ojo_e8r_quantize8 of w / s, then the MMSE scale
 *   sum(w * q) / clamp(sum(q * q), 1e-8)  with q = lut[code] (the x2 table),
 * both sums in torch's order; stored as fp16. */
static void e8r_encode_group(const float* w, int64_t gs, const float* lut, uint8_t* codes,
                             uint16_t* scale16, float* scale32) {
    float s = ojo_e8t_group_scale(w, gs);
    float prod[4096], qq[4096];
    for (int64_t t = 0; t < gs / 8; ++t) {
        float v[8];
        for (int i = 0; i < 8; ++i) v[i] = w[8 * t + i] / s;
        int32_t c = ojo_e8r_quantize8(v);
        codes[t] = (uint8_t)c;
        for (int i = 0; i < 8; ++i) {
            float q = lut[8 * c + i];
            prod[8 * t + i] = w[8 * t + i] * q;
            qq[8 * t + i] = q * q;
        }
    }
    float num = torch_row_sum(prod, gs);
    float den = torch_row_sum(qq, gs);
    if (den < 1e-8f) den = 1e-8f;
    float mm = num / den;
    *scale16 = ojo_f32_to_f16(mm);
    if (scale32) *scale32 = mm;
}

/* RootE8LatticePacker.pack on a flat fp32 array (gs a positive multiple of 8, at most
 * 4096; the caller applies the reference's coercion of other values to 8).
 * codes: padded/8 bytes; scales: padded/gs fp16 bits; scales32 optional. */
OJO_API void ojo_e8r_encode(const float* w, int64_t numel, int64_t gs, uint8_t* codes,
                            uint16_t* scales, float* scales32, int nthreads) {
    float lut[256 * 8];
    ojo_e8r_lut(lut);
    ojo_e8r_prepare();
    int64_t padded = ojo_e8t_padded(numel, gs);
    int64_t ngroups = padded / gs;
    int64_t full = numel / gs;
#ifdef _OPENMP
    if (nthreads <= 0) nthreads = omp_get_max_threads();
#pragma omp parallel for schedule(static) num_threads(nthreads)
#endif
    for (int64_t g = 0; g < full; ++g)
        e8r_encode_group(w + g * gs, gs, lut, codes + g * gs / 8, scales + g,
                         scales32 ? scales32 + g : 0);
    (void)nthreads;
    if (full < ngroups) { /* tail group, zero padded (F.pad, lattice.py:490-492) */
        float buf[4096];
        if (gs > 4096) return;
        int64_t rem = numel - full * gs;
        for (int64_t i = 0; i < gs; ++i) buf[i] = i < rem ? w[full * gs + i] : 0.0f;
        e8r_encode_group(buf, gs, lut, codes + full * gs / 8, scales + full,
                         scales32 ? scales32 + full : 0);
    }
}

/* Decoded weight as RootE8LatticePacker.unpack produces it (lattice.py:519-533):
 * lut.to(dtype)[code] * scales.to(dtype), the product rounded to dtype (coordinates
 * are 0, +-1, +-2: the fp32 product is exact).  gs = padded / numel(scales). */
OJO_API void ojo_e8r_decode(const uint8_t* codes, const uint16_t* scales, int64_t numel,
                            int64_t gs, int out_dtype, void* out) {
    float lut[256 * 8];
    ojo_e8r_lut(lut);
#ifdef _OPENMP
#pragma omp parallel for schedule(static)
#endif
    for (int64_t f = 0; f < numel; ++f) {
        float s = ojo_f16_to_f32(scales[f / gs]);
        if (out_dtype == 2) s = ojo_bf16_to_f32(ojo_f32_to_bf16(s));
        float p = lut[8 * codes[f >> 3] + (f & 7)] * s;
        if (out_dtype == 0) ((float*)out)[f] = p;
        else if (out_dtype == 1) ((uint16_t*)out)[f] = ojo_f32_to_f16(p);
        else ((uint16_t*)out)[f] = ojo_f32_to_bf16(p);
    }
}

static inline double e8r_deq(const float* lut, const uint8_t* codes, const uint16_t* scales,
                             int64_t f, int64_t gs, int w_dtype) {
    float s = ojo_f16_to_f32(scales[f / gs]);
    if (w_dtype == 2) s = ojo_bf16_to_f32(ojo_f32_to_bf16(s));
    float p = lut[8 * codes[f >> 3] + (f & 7)] * s;
    if (w_dtype == 1) p = ojo_f16_to_f32(ojo_f32_to_f16(p));
    else if (w_dtype == 2) p = ojo_bf16_to_f32(ojo_f32_to_bf16(p));
    return (double)p;
}

/* y = x . Wdeq^T + bias in fp64 (the reference's 1-bit forward: unpack + F.linear,
 * lattice.py:614-624).  Flat layout: element (n, k) is flat index n*K + k. */
OJO_API void ojo_e8r_gemm_f64(const float* x, const uint8_t* codes, const uint16_t* scales,
                              const float* bias, double* y, int64_t M, int64_t N, int64_t K,
                              int64_t gs, int w_dtype) {
    float lut[256 * 8];
    ojo_e8r_lut(lut);
#ifdef _OPENMP
#pragma omp parallel for schedule(static)
#endif
    for (int64_t n = 0; n < N; ++n) {
        for (int64_t m = 0; m < M; ++m) {
            double acc = bias ? (double)bias[n] : 0.0;
            for (int64_t k = 0; k < K; ++k)
                acc += (double)x[m * K + k] * e8r_deq(lut, codes, scales, n * K + k, gs, w_dtype);
            y[m * N + n] = acc;
        }
    }
}

/* grad_x = grad_y . Wdeq in fp64 (the portable backward, lattice.py:684-717). */
OJO_API void ojo_e8r_gemm_bwd_f64(const float* gy, const uint8_t* codes, const uint16_t* scales,
                                  double* gx, int64_t M, int64_t N, int64_t K, int64_t gs,
                                  int w_dtype) {
    float lut[256 * 8];
    ojo_e8r_lut(lut);
#ifdef _OPENMP
#pragma omp parallel for schedule(static)
#endif
    for (int64_t m = 0; m < M; ++m)
        for (int64_t k = 0; k < K; ++k) {
            double acc = 0.0;
            for (int64_t n = 0; n < N; ++n)
                acc += (double)gy[m * N + n] * e8r_deq(lut, codes, scales, n * K + k, gs, w_dtype);
            gx[m * K + k] = acc;
        }
}

OJO_API void ojo_e8r_quantize8_array(const float* v, int64_t nvec, int32_t* codes) {
    ojo_e8r_prepare();
#ifdef _OPENMP
#pragma omp parallel for schedule(static)
#endif
    for (int64_t i = 0; i < nvec; ++i) codes[i] = ojo_e8r_quantize8(v + 8 * i);
}

/* ------------------------------------------------------------------------- */
/* Conway-Sloane E8 projection and the QAT straight-through quantizer           */
/* ------------------------------------------------------------------------- */

/* conway_sloane_e8_project as its torch path computes it (lattice.py:180-203), for one
 * 8-vector, in fp32 (OJO_CS_T float) and fp64: the nearest point of D8 (round half to
 * even, parity fixed at the first largest rounding error, towards x) and of D8 + 1/2
 * (the same on x - 1/2, plus 1/2), the closer one by the sequential sum of squared
 * differences, D8 on ties. */
#define OJO_CS_DEFINE(NAME, T, RINT, FABS)                                              \
    static void NAME##_candidate(const T* x, T shift, T out[8]) {                       \
        T f[8], xs[8];                                                                  \
        long sum = 0;                                                                   \
        int worst = 0;                                                                  \
        T werr = 0;                                                                     \
        for (int i = 0; i < 8; ++i) {                                                   \
            xs[i] = x[i] - shift;                                                       \
            f[i] = RINT(xs[i]);                                                         \
            sum += (long)f[i];                                                          \
            T err = FABS(xs[i] - f[i]);                                                 \
            if (i == 0 || err > werr) { werr = err; worst = i; }                        \
        }                                                                               \
        if (sum % 2 != 0) {                                                             \
            T d = xs[worst] - f[worst];                                                 \
            f[worst] = f[worst] + ((d < 0) ? (T)-1 : (T)1);                             \
        }                                                                               \
        for (int i = 0; i < 8; ++i) out[i] = f[i] + shift;                              \
    }                                                                                   \
    OJO_API void NAME(const T* x, T* out, int64_t nvec) {                               \
        for (int64_t b = 0; b < nvec; ++b) {                                            \
            const T* v = x + 8 * b;                                                     \
            T c1[8], c2[8];                                                             \
            NAME##_candidate(v, (T)0, c1);                                              \
            NAME##_candidate(v, (T)0.5, c2);                                            \
            T d1 = 0, d2 = 0;                                                           \
            for (int i = 0; i < 8; ++i) {                                               \
                T a = v[i] - c1[i], b2 = v[i] - c2[i];                                  \
                T a2 = a * a, bb = b2 * b2;                                             \
                d1 = d1 + a2;                                                           \
                d2 = d2 + bb;                                                           \
            }                                                                           \
            const T* ch = (d1 <= d2) ? c1 : c2;                                         \
            for (int i = 0; i < 8; ++i) out[8 * b + i] = ch[i];                         \
        }                                                                               \
    }

OJO_CS_DEFINE(ojo_e8_cs_project_f32, float, rintf, fabsf)
OJO_CS_DEFINE(ojo_e8_cs_project_f64, double, rint, fabs)

/* The same projection on fp16 (half = 0) or bf16 (half = 1) tensors, as torch evaluates the
 * reference's expressions (lattice.py:180-203) on such a tensor: every elementwise op is
 * computed in fp32 and rounded to the tensor's type; a sum over the last dim adds the
 * fp32 values left to right and rounds once (the parity test reads that rounded sum, so a
 * sum that rounds to an even number counts as even); x - 0.5, the parity move f +- 1 and
 * c + 0.5 are each rounded, and so are x - c and its square.  Values are fp32 holding
 * exact half values; outputs too. */
static float ojo_rnd_half(float v, int half) {
    return half ? ojo_bf16_to_f32(ojo_f32_to_bf16(v)) : ojo_f16_to_f32(ojo_f32_to_f16(v));
}

static void ojo_cs_half_candidate(const float* x, int shifted, int half, float out[8]) {
    float f[8], xs[8];
    float sum = 0.0f;
    int worst = 0;
    float werr = 0.0f;
    for (int i = 0; i < 8; ++i) {
        xs[i] = shifted ? ojo_rnd_half(x[i] - 0.5f, half) : x[i];
        f[i] = rintf(xs[i]);
        sum = sum + f[i];
        float err = ojo_rnd_half(fabsf(xs[i] - f[i]), half);
        if (i == 0 || err > werr) { werr = err; worst = i; }
    }
    long isum = (long)ojo_rnd_half(sum, half);
    if (isum % 2 != 0) {
        float d = xs[worst] - f[worst];
        f[worst] = ojo_rnd_half(f[worst] + ((d < 0) ? -1.0f : 1.0f), half);
    }
    for (int i = 0; i < 8; ++i) out[i] = shifted ? ojo_rnd_half(f[i] + 0.5f, half) : f[i];
}

OJO_API void ojo_e8_cs_project_half(const float* x, float* out, int64_t nvec, int half) {
    for (int64_t b = 0; b < nvec; ++b) {
        const float* v = x + 8 * b;
        float c1[8], c2[8];
        ojo_cs_half_candidate(v, 0, half, c1);
        ojo_cs_half_candidate(v, 1, half, c2);
        float d1 = 0.0f, d2 = 0.0f;
        for (int i = 0; i < 8; ++i) {
            float a = ojo_rnd_half(v[i] - c1[i], half), bb = ojo_rnd_half(v[i] - c2[i], half);
            d1 = d1 + ojo_rnd_half(a * a, half);
            d2 = d2 + ojo_rnd_half(bb * bb, half);
        }
        d1 = ojo_rnd_half(d1, half);
        d2 = ojo_rnd_half(d2, half);
        const float* ch = (d1 <= d2) ? c1 : c2;
        for (int i = 0; i < 8; ++i) out[8 * b + i] = ch[i];
    }
}

/* _E8STEFunction.forward on fp16 / bf16 weights (fp32 holding exact half values), every op
 * rounded to the type: n = torch.norm(w8) (fp32 squares added left to right, sqrt, one
 * rounding), s = rnd(rnd(n / fp32(sqrt 8)) + fp32(1e-8)) (an fp16 zero vector gets s = 0
 * and NaN outputs, as the reference does), v = rnd(w / s), p = project(v) in the type,
 * out = rnd(p * s). */
OJO_API void ojo_e8_ste_quantize_half(const float* w, int64_t numel, float* out, int half) {
    int64_t nvec = (numel + 7) / 8;
    for (int64_t b = 0; b < nvec; ++b) {
        float x[8], v[8], p[8];
        for (int i = 0; i < 8; ++i) x[i] = (8 * b + i < numel) ? w[8 * b + i] : 0.0f;
        float acc = x[0] * x[0];
        for (int i = 1; i < 8; ++i) acc = acc + x[i] * x[i];
        float n = ojo_rnd_half(sqrtf(acc), half);
        float s = ojo_rnd_half(n / 2.8284271247461903f, half);
        s = ojo_rnd_half(s + 9.99999993922529e-09f, half);
        for (int i = 0; i < 8; ++i) v[i] = ojo_rnd_half(x[i] / s, half);
        ojo_e8_cs_project_half(v, p, 1, half);
        for (int i = 0; i < 8; ++i)
            if (8 * b + i < numel) out[8 * b + i] = ojo_rnd_half(p[i] * s, half);
    }
}

/* _E8STEFunction.forward (lattice.py:853-865) on fp32 weights: flat, zero padded to a
 * multiple of 8; per 8-vector s = torch.norm(w8)/sqrt(8) + 1e-8 (the CPU norm order),
 * out = project(w8 / s) * s; the first numel values. */
OJO_API void ojo_e8_ste_quantize_f32(const float* w, int64_t numel, float* out) {
    int64_t nvec = (numel + 7) / 8;
    for (int64_t b = 0; b < nvec; ++b) {
        float x[8], v[8], p[8];
        for (int i = 0; i < 8; ++i) x[i] = (8 * b + i < numel) ? w[8 * b + i] : 0.0f;
        float s = ojo_e8t_group_scale(x, 8);
        for (int i = 0; i < 8; ++i) v[i] = x[i] / s;
        ojo_e8_cs_project_f32(v, p, 1);
        for (int i = 0; i < 8; ++i)
            if (8 * b + i < numel) out[8 * b + i] = p[i] * s;
    }
}
