/*
 * nkv_oracle.c -- CPU restatement of NanoKV's codec arithmetic.
 *
 * TEST INFRASTRUCTURE ONLY.  This file is the checker that the HIP product
 * path is compared against.  Only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py may load it; the product library never links
 * it and never falls back to it.
 *
 * Every function restates one step of the reference algorithm and cites the
 * reference lines it follows (paths relative to the NanoKV source tree):
 *
 *   MG  = models/Matrix-Game-3.5/fast/diffsynth/models/nanokv_codec.py
 *   HY  = models/HY-WorldPlay/compression/hyvideo/models/transformers/modules/kv_codecs.py
 *   HYT = models/HY-WorldPlay/compression/hyvideo/models/transformers/modules/kv_codec_triton.py
 *   LK  = models/Matrix-Game-3.5/fast/codec_native/latent_kernel.py
 *
 * Written in plain C99 so that each floating-point operation happens exactly
 * once, in the stated precision, with no contraction (build with
 * -ffp-contract=off).  Pinning of each function (the independent checks that
 * make it trustworthy) is listed in the header comment of oracle/oracle.py.
 */
#include <math.h>
#include <stdint.h>
#include <string.h>
#include <float.h>

/* ------------------------------------------------------------------ */
/* IEEE conversions (round to nearest even).                            */
/* ------------------------------------------------------------------ */

static inline uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

/* float -> bfloat16 bits, round-to-nearest-even; NaN stays a quiet NaN.
 * torch's Tensor.to(torch.bfloat16) has the same contract (MG:333-365 casts
 * scales, centers and decoded rows this way). */
uint16_t nkvo_f32_to_bf16(float f) {
    uint32_t u = f2u(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x0040u);
    uint32_t lsb = (u >> 16) & 1u;
    u += 0x7fffu + lsb;
    return (uint16_t)(u >> 16);
}

float nkvo_bf16_to_f32(uint16_t h) { return u2f(((uint32_t)h) << 16); }

static inline float bf16_round(float f) { return nkvo_bf16_to_f32(nkvo_f32_to_bf16(f)); }

/* float -> IEEE binary16 bits, round-to-nearest-even, with subnormals,
 * overflow to +-inf and NaN preserved (torch's .to(torch.float16)). */
uint16_t nkvo_f32_to_f16(float f) {
    uint32_t u = f2u(f);
    uint32_t sign = (u >> 16) & 0x8000u;
    uint32_t absu = u & 0x7fffffffu;
    if (absu > 0x7f800000u) return (uint16_t)(sign | 0x7e00u);          /* NaN */
    if (absu >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u);         /* >= 65520 rounds to inf */
    if (absu < 0x38800000u) {                                           /* below 2^-14: subnormal or zero */
        /* value = absu as float; subnormal unit is 2^-24. */
        float a = u2f(absu);
        /* a * 2^24 is exact in float (power-of-two scaling, no overflow). */
        float scaled = a * 16777216.0f;
        /* round half to even to an integer count of 2^-24 units. */
        float r = rintf(scaled);
        return (uint16_t)(sign | (uint32_t)r);                          /* r <= 1024 -> may become min normal */
    }
    /* normal range: rebias exponent 127 -> 15 and round 23 -> 10 mantissa bits. */
    uint32_t mant = absu & 0x7fffffu;
    uint32_t exp = (absu >> 23) - 127 + 15;
    uint32_t h = (exp << 10) | (mant >> 13);
    uint32_t rem = mant & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h += 1;          /* carry may bump the exponent: correct */
    return (uint16_t)(sign | h);
}

float nkvo_f16_to_f32(uint16_t h) {
    uint32_t sign = ((uint32_t)h & 0x8000u) << 16;
    uint32_t exp = (h >> 10) & 0x1fu;
    uint32_t mant = h & 0x3ffu;
    if (exp == 0) {
        float v = (float)mant * (1.0f / 16777216.0f);                   /* mant * 2^-24, exact */
        return sign ? -v : v;
    }
    if (exp == 31) return u2f(sign | 0x7f800000u | (mant << 13));
    return u2f(sign | ((exp - 15 + 127) << 23) | (mant << 13));
}

static inline float scale_decode(uint16_t bits, int scale_dtype) {
    return scale_dtype == 1 ? nkvo_f16_to_f32(bits) : nkvo_bf16_to_f32(bits);
}

static inline uint16_t scale_encode(float s, int scale_dtype) {
    return scale_dtype == 1 ? nkvo_f32_to_f16(s) : nkvo_f32_to_bf16(s);
}

/* ------------------------------------------------------------------ */
/* a4 + a5: INT4 quantisation and packing.                              */
/* ------------------------------------------------------------------ */

/*
 * Quantise fp32 coefficients [rows, r] in scale groups of `group` columns and
 * pack two codes per byte.
 *
 * quant_mode 0 (fp32 arithmetic) follows HY:237-255 (`per_token`) and the
 * MG:349-351 formula with fp32 operands:
 *     s     = max(amax|x|, FLT_EPSILON) / 7          (fp32, IEEE division)
 *     code  = clamp(round_half_even(x / s), -7, 7)   (fp32 division)
 *     store = cast(s) to bf16 (scale_dtype 0) or fp16 (scale_dtype 1)
 * Codes use the unrounded s; decode uses the stored s (MG:349-351, 426-434).
 *
 * quant_mode 1 (bf16 arithmetic) follows MG:349-351 as deployed, where
 * `coeff` is a bf16 tensor (MG:138-153 returns bf16 for int8/bf16
 * operators): every elementwise op computes in fp32 and rounds to bf16:
 *     a = bf16(max(amax, eps));  s = bf16(a / 7);  q = bf16(x / s)
 *     code = clamp(round_half_even(q), -7, 7);     store = cast(s)
 * The input x is rounded to bf16 first in this mode.
 *
 * Group g of a row spans columns [g*group, (g+1)*group); group == r gives the
 * reference's one-scale-per-row layout.  Scales are [rows, r/group].
 *
 * Packing follows MG:282-292: over the row-major flattened codes,
 * byte j = (c[2j] + 7) | ((c[2j+1] + 7) << 4).  r must be even, so rows
 * never share a byte.
 */
void nkvo_quant_pack(const float* coeff, int64_t rows, int r, int group,
                     int scale_dtype, int quant_mode,
                     uint8_t* packed, uint16_t* scales, int8_t* codes_out) {
    int ngroups = r / group;
    for (int64_t row = 0; row < rows; ++row) {
        const float* x = coeff + row * (int64_t)r;
        for (int g = 0; g < ngroups; ++g) {
            const float* xg = x + (int64_t)g * group;
            float amax = 0.0f;
            for (int j = 0; j < group; ++j) {
                float v = quant_mode == 1 ? bf16_round(xg[j]) : xg[j];
                float a = fabsf(v);
                if (a > amax || isnan(a)) amax = a;    /* amax propagates NaN like torch */
            }
            float s;
            if (quant_mode == 1) {
                float a = bf16_round(amax > FLT_EPSILON || isnan(amax) ? amax : FLT_EPSILON);
                s = bf16_round(a / 7.0f);
            } else {
                float a = (amax > FLT_EPSILON || isnan(amax)) ? amax : FLT_EPSILON;
                s = a / 7.0f;
            }
            scales[row * ngroups + g] = scale_encode(s, scale_dtype);
            for (int j = 0; j < group; ++j) {
                float v = quant_mode == 1 ? bf16_round(xg[j]) : xg[j];
                float q = v / s;
                if (quant_mode == 1) q = bf16_round(q);
                float rq = rintf(q);                   /* round half to even (torch.round) */
                int c;
                if (isnan(rq)) c = 0;                  /* not part of the contract; keep deterministic */
                else if (rq > 7.0f) c = 7;
                else if (rq < -7.0f) c = -7;
                else c = (int)rq;
                int col = g * group + j;
                if (codes_out) codes_out[row * (int64_t)r + col] = (int8_t)c;
                uint8_t nib = (uint8_t)(c + 7);
                int64_t byte = row * (int64_t)(r / 2) + col / 2;
                if ((col & 1) == 0) packed[byte] = nib;
                else packed[byte] = (uint8_t)(packed[byte] | (nib << 4));
            }
        }
    }
}

/* a5 inverse: MG:295-298 -- low nibble is the even index; code = nibble - 7. */
void nkvo_unpack_codes(const uint8_t* packed, int64_t count, int8_t* codes) {
    for (int64_t i = 0; i < count; ++i) {
        uint8_t b = packed[i >> 1];
        int nib = (i & 1) ? (b >> 4) : (b & 15);
        codes[i] = (int8_t)(nib - 7);
    }
}

/*
 * a7: INT4 unpack x scale -> bf16 latent.  MG:426-434 (CPU: fp32 product,
 * rounded to bf16 at the F.linear input MG:138-141) and the CUDA kernel
 * nanokv_codec_kernels.py:11-27 (fp32 product stored to a bf16 tensor):
 *     latent[n, j] = bf16( float(code) * float(stored_scale[n, j / group]) )
 * `row_index` (may be NULL) selects source rows as LK:7-23 does.
 */
void nkvo_unpack_latent(const uint8_t* packed, const uint16_t* scales,
                        int scale_dtype, const int32_t* row_index, int64_t rows,
                        int r, int group, uint16_t* out) {
    int ngroups = r / group;
    for (int64_t i = 0; i < rows; ++i) {
        int64_t src = row_index ? (int64_t)row_index[i] : i;
        for (int j = 0; j < r; ++j) {
            uint8_t b = packed[src * (int64_t)(r / 2) + j / 2];
            int nib = (j & 1) ? (b >> 4) : (b & 15);
            float s = scale_decode(scales[src * ngroups + j / group], scale_dtype);
            out[i * (int64_t)r + j] = nkvo_f32_to_bf16((float)(nib - 7) * s);
        }
    }
}

/* ------------------------------------------------------------------ */
/* a1: nearest-center assignment.                                       */
/* ------------------------------------------------------------------ */

/*
 * ids[n] = argmin_c ||x_n - c||^2 over the given bf16 center table, first
 * index on ties.  The reference evaluates the expansion
 * ||x||^2 + ||c||^2 - 2 x.c in fp32 with a bmm (MG:315-321, HY:146-152) whose
 * reduction order is library-defined; this restatement fixes the order-free
 * answer by evaluating ||c||^2 - 2 x.c in fp64 (||x||^2 is constant per row
 * and cannot change the argmin).  Every product of an fp32 x and a bf16 c is
 * exact in fp64, so only the fp64 summation rounds (relative 1e-16).
 */
void nkvo_assign(const float* x, const uint16_t* centers, int64_t rows, int C,
                 int HD, int32_t* ids) {
    for (int64_t n = 0; n < rows; ++n) {
        const float* xr = x + n * (int64_t)HD;
        double best = 0.0;
        int best_c = 0;
        for (int c = 0; c < C; ++c) {
            const uint16_t* cr = centers + (int64_t)c * HD;
            double cc = 0.0, xc = 0.0;
            for (int k = 0; k < HD; ++k) {
                double cv = (double)nkvo_bf16_to_f32(cr[k]);
                cc += cv * cv;
                xc += (double)xr[k] * cv;
            }
            double d = cc - 2.0 * xc;
            if (c == 0 || d < best) { best = d; best_c = c; }
        }
        ids[n] = best_c;
    }
}

/*
 * a1 residual: MG:326-330 and HY:191-200 -- x - fp32(bf16 center[id]) in
 * fp32, then the encoder input subtracts the fp32 mean (MG:346) and the
 * operator casts the result to bf16 (MG:138-141).  Returns bf16 bits.
 */
void nkvo_residual_bf16(const float* x, const uint16_t* centers, const int32_t* ids,
                        const float* mean, int64_t rows, int HD, uint16_t* out) {
    for (int64_t n = 0; n < rows; ++n) {
        const uint16_t* cr = centers ? centers + (int64_t)ids[n] * HD : NULL;
        for (int k = 0; k < HD; ++k) {
            float v = x[n * (int64_t)HD + k];
            if (cr) v = v - nkvo_bf16_to_f32(cr[k]);
            if (mean) v = v - mean[k];
            out[n * (int64_t)HD + k] = nkvo_f32_to_bf16(v);
        }
    }
}

/* ------------------------------------------------------------------ */
/* a8: decode epilogue rounding chain.                                  */
/* ------------------------------------------------------------------ */

/*
 * Given the fp32 decoder GEMM accumulator acc[n, k] = sum_j latent[n,j] *
 * W_dec[k,j] (bf16 operands), apply the reference's rounding points:
 *   rows = bf16(acc + float(bf16(mean)))      F.linear with bf16 bias,
 *                                             MG:138-141, 439-443
 *   rows = bf16(float(rows) + float(center))  MG:445-454 (`add_` of an fp32
 *                                             gather into a bf16 tensor);
 *                                             LK:26-52 casts the center to
 *                                             bf16 first -- same value, the
 *                                             center is bf16 already.
 * `centers`/`ids` may be NULL (pca rung, MG:334-341 `semantic=False`).
 * `mean` may be NULL (zero bias).
 */
void nkvo_decode_epilogue(const float* acc, const float* mean,
                          const uint16_t* centers, const int32_t* ids,
                          int64_t rows, int HD, uint16_t* out) {
    for (int64_t n = 0; n < rows; ++n) {
        for (int k = 0; k < HD; ++k) {
            float b = mean ? bf16_round(mean[k]) : 0.0f;
            float v = bf16_round(acc[n * (int64_t)HD + k] + b);
            if (centers) v = bf16_round(v + nkvo_bf16_to_f32(centers[(int64_t)ids[n] * HD + k]));
            out[n * (int64_t)HD + k] = nkvo_f32_to_bf16(v);
        }
    }
}

/* Round an fp32 array to bf16 bits (for the fixtures and tests). */
void nkvo_round_bf16(const float* x, int64_t n, uint16_t* out) {
    for (int64_t i = 0; i < n; ++i) out[i] = nkvo_f32_to_bf16(x[i]);
}

void nkvo_round_f16(const float* x, int64_t n, uint16_t* out) {
    for (int64_t i = 0; i < n; ++i) out[i] = nkvo_f32_to_f16(x[i]);
}

void nkvo_widen_bf16(const uint16_t* x, int64_t n, float* out) {
    for (int64_t i = 0; i < n; ++i) out[i] = nkvo_bf16_to_f32(x[i]);
}

void nkvo_widen_f16(const uint16_t* x, int64_t n, float* out) {
    for (int64_t i = 0; i < n; ++i) out[i] = nkvo_f16_to_f32(x[i]);
}


/* INT8 operator storage, _pack_operator (MG:108-131): per (row, group)
 * s = max(amax|w|, 1e-12) / 127 in fp32, q = clamp(rint(w / s), -127, 127),
 * scale = bf16(s). */
void nkvo_int8_pack(const float* w, int64_t rows, int cols, int group, int8_t* q,
                    uint16_t* scale) {
    int ngroups = cols / group;
    for (int64_t row = 0; row < rows; ++row) {
        for (int g = 0; g < ngroups; ++g) {
            const float* wg = w + row * (int64_t)cols + (int64_t)g * group;
            float amax = 0.0f;
            for (int j = 0; j < group; ++j) {
                float a = fabsf(wg[j]);
                if (a > amax || isnan(a)) amax = a;
            }
            float s = (amax > 1e-12f || isnan(amax) ? amax : 1e-12f) / 127.0f;
            scale[row * ngroups + g] = nkvo_f32_to_bf16(s);
            for (int j = 0; j < group; ++j) {
                float r = rintf(wg[j] / s);
                if (isnan(r)) r = -127.0f;             /* as fmax(NaN, -127) */
                if (r > 127.0f) r = 127.0f;
                if (r < -127.0f) r = -127.0f;
                q[row * (int64_t)cols + (int64_t)g * group + j] = (int8_t)(int)r;
            }
        }
    }
}

/* bf16(q * scale) of every weight (unpack_int8_weight,
 * nanokv_codec_kernels.py:64-82). */
void nkvo_int8_dequant(const int8_t* q, const uint16_t* scale, int64_t rows, int cols, int group,
                       uint16_t* out) {
    for (int64_t i = 0; i < rows * (int64_t)cols; ++i)
        out[i] = nkvo_f32_to_bf16((float)q[i] * nkvo_bf16_to_f32(scale[i / group]));
}
