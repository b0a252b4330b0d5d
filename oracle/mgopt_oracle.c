/*
 * mgopt_oracle.c -- CPU oracle for the fused optimizer step.
 *
 * TEST INFRASTRUCTURE ONLY.  Nothing in the product loads this library; only
 * tests/, __graft_entry__.smoke() and the cpu_baseline leg of bench.py do, and
 * only as the reference results that the GPU path is compared against.
 *
 * What it restates.  The reference's training loop runs, once per iteration
 * (train.py:483-491):
 *
 *     scaler.unscale_(optimizer)
 *     grad_norm = torch.nn.utils.clip_grad_norm_(model.parameters(), grad_clip)
 *     scaler.step(optimizer)
 *     scaler.update()
 *
 * with torch.optim.AdamW built at train.py:359-365 and torch.amp.GradScaler
 * at train.py:366-370.  All arithmetic on that path lives in the reference's
 * pinned third-party dependency, torch 2.10.0 (.github/workflows/
 * v06-frozen-review.yml:51-53; pyproject.toml:7 asks for torch>=2.8), not in
 * the reference's own files.  Each function below names the torch Python
 * source line it follows (paths relative to the torch package) and the
 * element-level rounding of the ATen CPU kernel that line dispatches to.  The
 * rounding choices were fixed by comparing against torch 2.10.0 CPU outputs;
 * tests/test_oracle_pinning.py keeps that comparison running.
 *
 * Two deliberate departures from torch's CPU path, both stated in tests:
 *   - sqrt is IEEE correctly rounded (sqrtf).  torch's CPU sqrt for large
 *     tensors goes through a vector math library that is off by one ulp on
 *     about 0.6% of inputs.
 *   - the gradient norm accumulates squares in fp64 with Neumaier
 *     compensation.  torch's CPU vector_norm accumulates each tensor in fp32
 *     sequentially, whose relative error grows with tensor size (about 3e-5
 *     at 2M elements, 2e-3 at 38.6M).
 *
 * Pinning.  Every restated function is checked by tests that a plausible
 * mistake fails, so none is "parity unpinned":
 *   - against torch 2.10.0 CPU golden vectors (tests/golden/, written by
 *     tests/golden/make_golden.py) and torch's CPU path run live on 40 seeded
 *     configurations (tests/test_oracle_random.py);
 *   - against closed forms (first step, zero gradient, bias corrections, exact
 *     rational norms, cosine schedule values, the scaler trajectory);
 *   - with six planted mistakes in the AdamW restatement, each rejected
 *     (tests/test_oracle_pinning.py).
 * orc_synth_value is the test-data generator, not reference arithmetic: it is
 * pinned against the GPU generator bit for bit (tests/test_gpu_parity.py).
 *
 * Build: oracle/Makefile (gcc -O3 -mfma -ffp-contract=off: the compiler forms
 * no fused multiply-add of its own, so every one below is an explicit fmaf).
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

#define ORC_API __attribute__((visibility("default")))

/* ------------------------------------------------------------------------- */
/* Scalar conversions                                                         */
/* ------------------------------------------------------------------------- */

static inline uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

/* float -> bfloat16, round to nearest even; every NaN becomes 0x7FC0.
 * Same rule as torch's Tensor.to(torch.bfloat16). */
ORC_API uint16_t orc_f32_to_bf16(float f) {
    uint32_t u = f2u(f);
    if (isnan(f)) return 0x7FC0u;
    uint32_t bias = 0x7FFFu + ((u >> 16) & 1u);
    return (uint16_t)((u + bias) >> 16);
}

ORC_API float orc_bf16_to_f32(uint16_t h) { return u2f((uint32_t)h << 16); }

/* float -> IEEE binary16, round to nearest even, with subnormals, overflow to
 * inf and NaN kept quiet.  Written from the binary16 definition. */
ORC_API uint16_t orc_f32_to_f16(float f) {
    uint32_t u = f2u(f);
    uint32_t sign = (u >> 16) & 0x8000u;
    uint32_t a = u & 0x7FFFFFFFu;
    if (a > 0x7F800000u) return (uint16_t)(sign | 0x7E00u | ((a >> 13) & 0x3FFu));
    if (a >= 0x477FF000u) return (uint16_t)(sign | 0x7C00u); /* >= 65520 rounds to inf */
    if (a < 0x38800000u) {
        /* result is subnormal or zero: value = a_real / 2^-24, rounded to int */
        if (a < 0x33000000u) return (uint16_t)sign; /* < 2^-25: rounds to 0 */
        uint32_t e = a >> 23;
        uint32_t mant = (a & 0x7FFFFFu) | 0x800000u;
        uint32_t shift = 126u - e; /* 2^(e-127) * mant/2^23 / 2^-24 = mant >> (126-e) ... */
        /* value/2^-24 = mant * 2^(e-127-23+24) = mant >> (126 - e) */
        uint32_t q = mant >> shift;
        uint32_t rem = mant & ((1u << shift) - 1u);
        uint32_t half = 1u << (shift - 1u);
        if (rem > half || (rem == half && (q & 1u))) q++;
        return (uint16_t)(sign | q);
    }
    /* normal range: rebias exponent 127 -> 15, round mantissa 23 -> 10 bits */
    uint32_t r = a - 0x38000000u; /* subtract (127-15) << 23 */
    uint32_t q = r >> 13;
    uint32_t rem = r & 0x1FFFu;
    if (rem > 0x1000u || (rem == 0x1000u && (q & 1u))) q++;
    return (uint16_t)(sign | q);
}

ORC_API float orc_f16_to_f32(uint16_t h) {
    uint32_t sign = ((uint32_t)h & 0x8000u) << 16;
    uint32_t e = ((uint32_t)h >> 10) & 0x1Fu;
    uint32_t m = (uint32_t)h & 0x3FFu;
    if (e == 0x1Fu) return u2f(sign | 0x7F800000u | (m << 13));
    if (e == 0) {
        float v = (float)m * 5.9604644775390625e-08f; /* m * 2^-24, exact */
        return sign ? -v : v;
    }
    return u2f(sign | ((e + 112u) << 23) | (m << 13));
}

ORC_API void orc_f32_to_bf16_array(const float* in, uint16_t* out, int64_t n) {
    for (int64_t i = 0; i < n; i++) out[i] = orc_f32_to_bf16(in[i]);
}
ORC_API void orc_bf16_to_f32_array(const uint16_t* in, float* out, int64_t n) {
    for (int64_t i = 0; i < n; i++) out[i] = orc_bf16_to_f32(in[i]);
}
ORC_API void orc_f32_to_f16_array(const float* in, uint16_t* out, int64_t n) {
    for (int64_t i = 0; i < n; i++) out[i] = orc_f32_to_f16(in[i]);
}
ORC_API void orc_f16_to_f32_array(const uint16_t* in, float* out, int64_t n) {
    for (int64_t i = 0; i < n; i++) out[i] = orc_f16_to_f32(in[i]);
}

/* ------------------------------------------------------------------------- */
/* Synthetic data (test inputs; no reference counterpart)                     */
/* ------------------------------------------------------------------------- */

static inline uint64_t mix64(uint64_t x) {
    x = (x ^ (x >> 30)) * 0xBF58476D1CE4E5B9ull;
    x = (x ^ (x >> 27)) * 0x94D049BB133111EBull;
    return x ^ (x >> 31);
}

#define SYNTH_GAMMA 0x9E3779B97F4A7C15ull

ORC_API uint64_t orc_synth_key(uint64_t seed, uint64_t stream) {
    return mix64(seed * SYNTH_GAMMA + mix64(stream + SYNTH_GAMMA));
}

/* Element idx of stream `key`: four 16-bit uniforms summed (Irwin-Hall, n=4),
 * centred, times k (= sigma*sqrt(3)/65536 gives variance sigma^2).  When
 * tail_every > 0, elements whose second hash is 0 mod tail_every are further
 * multiplied by tail_mult.  All arithmetic is integer or one IEEE double
 * product and one double->float rounding, so CPU and GPU agree bit for bit. */
ORC_API float orc_synth_value(uint64_t key, uint64_t idx, double k, uint64_t tail_every, double tail_mult) {
    uint64_t h = mix64(key + (idx + 1ull) * SYNTH_GAMMA);
    int32_t s = (int32_t)(h & 0xFFFFu) + (int32_t)((h >> 16) & 0xFFFFu) +
                (int32_t)((h >> 32) & 0xFFFFu) + (int32_t)(h >> 48) - 131070;
    double x = (double)s * k;
    if (tail_every) {
        uint64_t h2 = mix64(h ^ 0xD1B54A32D192ED03ull);
        if (h2 % tail_every == 0) x = x * tail_mult;
    }
    return (float)x;
}

ORC_API void orc_synth_fill(float* out, int64_t n, uint64_t seed, uint64_t stream, double k,
                            uint64_t tail_every, double tail_mult) {
    uint64_t key = orc_synth_key(seed, stream);
    for (int64_t i = 0; i < n; i++) out[i] = orc_synth_value(key, (uint64_t)i, k, tail_every, tail_mult);
}

/* The synthetic gradient of one tensor as the GPU holds it: elements
 * [begin, end) of stream (seed, stream), stored in dtype (0 fp32, 1 fp16,
 * 2 bf16; mgopt_synth_fill rounds to it) and read back as fp32. */
static inline float synth_grad_value(uint64_t key, uint64_t i, double k, uint64_t tail_every, double tail_mult,
                                     int dtype) {
    float x = orc_synth_value(key, i, k, tail_every, tail_mult);
    if (dtype == 1) return orc_f16_to_f32(orc_f32_to_f16(x));
    if (dtype == 2) return orc_bf16_to_f32(orc_f32_to_bf16(x));
    return x;
}

ORC_API void orc_synth_grad(float* out, int64_t begin, int64_t end, uint64_t seed, uint64_t stream, double k,
                            uint64_t tail_every, double tail_mult, int dtype) {
    uint64_t key = orc_synth_key(seed, stream);
    for (int64_t i = begin; i < end; i++)
        out[i - begin] = synth_grad_value(key, (uint64_t)i, k, tail_every, tail_mult, dtype);
}

/* ------------------------------------------------------------------------- */
/* a5: GradScaler.unscale_                                                    */
/* ------------------------------------------------------------------------- */

/* torch/amp/grad_scaler.py:336-340 computes inv_scale = float(1/double(scale)). */
ORC_API float orc_inv_scale(float scale) { return (float)(1.0 / (double)scale); }

/* torch/amp/grad_scaler.py:280-284 -> torch._amp_foreach_non_finite_check_and_unscale_:
 * a non-finite input element sets found_inf to 1.0; every element becomes
 * in * inv_scale (left as is when inv_scale == 1). */
ORC_API void orc_unscale(const float* in, float* out, int64_t n, float inv_scale, float* found_inf) {
    for (int64_t i = 0; i < n; i++) {
        float x = in[i];
        if (!isfinite(x)) *found_inf = 1.0f;
        out[i] = (inv_scale == 1.0f) ? x : x * inv_scale;
    }
}

/* ------------------------------------------------------------------------- */
/* a6: clip_grad_norm_                                                        */
/* ------------------------------------------------------------------------- */

/* Sum of squares of one tensor's gradient (torch/nn/utils/clip_grad.py:96,
 * per-tensor _foreach_norm before the square root).  Squares of floats are
 * exact in double; the running sum is Neumaier-compensated. The compensated
 * sum and its correction term are returned through acc[0..1] so that several
 * tensors can be chained. */
ORC_API void orc_sumsq_acc(const float* g, int64_t n, double* acc) {
    double s = acc[0], c = acc[1];
    for (int64_t i = 0; i < n; i++) {
        double x = (double)g[i];
        double y = x * x;
        double t = s + y;
        if (!isfinite(t)) {
            /* an inf square makes the sum inf, a NaN makes it NaN; the
             * correction term would turn inf into NaN, so it is dropped */
            s = t;
            c = 0.0;
            continue;
        }
        if (fabs(s) >= fabs(y)) c += (s - t) + y;
        else c += (y - t) + s;
        s = t;
    }
    acc[0] = s;
    acc[1] = c;
}

/* The unscale step followed by the sum of squares, over one gradient stored
 * as fp32 (dtype 0), fp16 (1) or bf16 (2): each element x is widened to
 * fp32, tested for finiteness (sets *found to 1), multiplied by inv when
 * unscale is nonzero (grad_scaler.py:280-284) and its square accumulated into
 * acc[0..1] as orc_sumsq_acc does (clip_grad.py:96). */
ORC_API void orc_grad_sumsq_acc(const void* data, int dtype, int64_t n, float inv, int unscale, double* acc,
                                float* found) {
    double s = acc[0], c = acc[1];
    const float* f = (const float*)data;
    const uint16_t* h = (const uint16_t*)data;
    for (int64_t i = 0; i < n; i++) {
        float x = dtype == 0 ? f[i] : (dtype == 1 ? orc_f16_to_f32(h[i]) : orc_bf16_to_f32(h[i]));
        if (!isfinite(x)) *found = 1.0f;
        if (unscale && inv != 1.0f) x = x * inv;
        double y = (double)x * (double)x;
        double t = s + y;
        if (!isfinite(t)) {
            s = t;
            c = 0.0;
            continue;
        }
        if (fabs(s) >= fabs(y)) c += (s - t) + y;
        else c += (y - t) + s;
        s = t;
    }
    acc[0] = s;
    acc[1] = c;
}

/* orc_grad_sumsq_acc over elements [begin, end) of a synthetic gradient
 * (orc_synth_grad), generated on the fly instead of read from memory. */
ORC_API void orc_synth_grad_sumsq_acc(int64_t begin, int64_t end, uint64_t seed, uint64_t stream, double k,
                                      uint64_t tail_every, double tail_mult, int dtype, float inv, int unscale,
                                      double* acc, float* found) {
    uint64_t key = orc_synth_key(seed, stream);
    double s = acc[0], c = acc[1];
    for (int64_t i = begin; i < end; i++) {
        float x = synth_grad_value(key, (uint64_t)i, k, tail_every, tail_mult, dtype);
        if (!isfinite(x)) *found = 1.0f;
        if (unscale && inv != 1.0f) x = x * inv;
        double y = (double)x * (double)x;
        double t = s + y;
        if (!isfinite(t)) {
            s = t;
            c = 0.0;
            continue;
        }
        if (fabs(s) >= fabs(y)) c += (s - t) + y;
        else c += (y - t) + s;
        s = t;
    }
    acc[0] = s;
    acc[1] = c;
}

ORC_API double orc_sumsq(const float* g, int64_t n) {
    double acc[2] = {0.0, 0.0};
    orc_sumsq_acc(g, n, acc);
    return acc[0] + acc[1];
}

/* Total norm from the total sum of squares (clip_grad.py:106-108: the norm
 * of the stacked per-tensor norms equals sqrt of the summed squares).  A sum
 * that overflows fp32 gives inf, as torch's fp32 accumulation does. NaN stays
 * NaN; an infinite element gives inf. */
ORC_API float orc_norm_from_sumsq(double s) {
    if (isnan(s)) return NAN;
    if (isinf((float)s)) return INFINITY;
    return (float)sqrt(s);
}

/* clip_grad.py:165-169: clip_coef = max_norm / (total_norm + 1e-6), which
 * torch evaluates as reciprocal(total_norm + 1e-6) * max_norm
 * (torch/_tensor.py:1119-1122), then clamp(max=1.0).  NaN propagates. */
ORC_API float orc_clip_coef(float total_norm, float max_norm) {
    float d = total_norm + 1e-6f;
    float r = 1.0f / d;
    float c = r * max_norm;
    if (isnan(c)) return c;
    return c > 1.0f ? 1.0f : c;
}

/* clip_grad.py:174: _foreach_mul_(grads, clip_coef_clamped). */
ORC_API void orc_scale(float* g, int64_t n, float coef) {
    for (int64_t i = 0; i < n; i++) g[i] = g[i] * coef;
}

/* ------------------------------------------------------------------------- */
/* a8: AdamW, single-tensor CPU path                                          */
/* ------------------------------------------------------------------------- */

/* Host-double scalars exactly as torch/optim/adam.py:529-536 forms them from
 * step = state["step"].item() (a Python float). out[0] = bias_correction1,
 * out[1] = bias_correction2 ** 0.5. */
ORC_API void orc_bias_corrections(double beta1, double beta2, double step, double* out) {
    out[0] = 1.0 - pow(beta1, step);
    out[1] = pow(1.0 - pow(beta2, step), 0.5);
}

/* One AdamW update of one tensor, after step_t += 1 (adam.py:414), given the
 * new step value.  Element order and rounding:
 *   adam.py:416-419  p = p * float(1 - lr*wd)                (if wd != 0)
 *   adam.py:457      m.lerp_(g, 1 - beta1): ATen's vector lerp,
 *                    fma(w, g - m, m) for |w| < 0.5, else fma(w - 1, g - m, g)
 *   adam.py:476      v = v * float(beta2); v = fma(float(1-beta2) * g, g, v)
 *   adam.py:542      d = sqrt(v) / float(bc2 ** 0.5) + float(eps)
 *   adam.py:547      p = p + (float(-lr/bc1) * m) / d
 * maximize negates the gradient first (adam.py:397). */
ORC_API void orc_adamw(float* p, const float* g, float* m, float* v, int64_t n,
                       double lr, double beta1, double beta2, double eps, double wd,
                       double step, int maximize) {
    double bc[2];
    orc_bias_corrections(beta1, beta2, step, bc);
    const double step_size = lr / bc[0];
    const float decay = (float)(1.0 - lr * wd);
    const float w1 = (float)(1.0 - beta1);
    const float w1m1 = w1 - 1.0f;
    const int small = fabsf(w1) < 0.5f;
    const float b2 = (float)beta2;
    const float w2 = (float)(1.0 - beta2);
    const float bc2s = (float)bc[1];
    const float epsf = (float)eps;
    const float nss = (float)(-step_size);
    for (int64_t i = 0; i < n; i++) {
        float gi = maximize ? -g[i] : g[i];
        float pi = p[i];
        if (wd != 0.0) pi = pi * decay;
        float mi = m[i];
        float diff = gi - mi;
        mi = small ? fmaf(w1, diff, mi) : fmaf(w1m1, diff, gi);
        float vi = v[i] * b2;
        float sg = w2 * gi;
        vi = fmaf(sg, gi, vi);
        float d = sqrtf(vi);
        d = d / bc2s;
        d = d + epsf;
        float u = nss * mi;
        u = u / d;
        pi = pi + u;
        p[i] = pi;
        m[i] = mi;
        v[i] = vi;
    }
}

/* One tensor's share of an iteration whose step is taken, as OracleRun.step
 * performs it: orc_unscale (when `unscale`), then orc_scale by the clip
 * coefficient (when `clip`), then orc_adamw.  The tensor is processed in
 * blocks of ORC_BLOCK elements through a stack buffer, each block through
 * exactly those three functions, so the result is bit for bit that of the
 * three calls over the whole tensor (tests/test_oracle_pinning.py checks
 * it); the blocking keeps the unscaled gradient in cache instead of in a
 * tensor-sized array. */
#define ORC_BLOCK 2048
ORC_API void orc_unscale_clip_adamw(const float* g, float* p, float* m, float* v, int64_t n,
                                    float inv, int unscale, float coef, int clip,
                                    double lr, double beta1, double beta2, double eps, double wd,
                                    double step, int maximize) {
    float buf[ORC_BLOCK];
    float found = 0.0f;
    for (int64_t s = 0; s < n; s += ORC_BLOCK) {
        const int64_t k = n - s < ORC_BLOCK ? n - s : ORC_BLOCK;
        if (unscale) orc_unscale(g + s, buf, k, inv, &found);
        else memcpy(buf, g + s, (size_t)k * sizeof(float));
        if (clip) orc_scale(buf, k, coef);
        orc_adamw(p + s, buf, m + s, v + s, k, lr, beta1, beta2, eps, wd, step, maximize);
    }
}

/* Deliberately wrong variants of orc_adamw, used only by the pinning tests to
 * show that the golden checks reject plausible mistakes:
 *   1: drops the bias correction of the first moment
 *   2: uses beta2 where 1 - beta2 belongs in the second moment
 *   3: applies weight decay after the Adam update instead of before
 *   4: flips the sign of the update
 *   5: rounds the lerp as two operations instead of one fused multiply-add
 *   6: sqrt(v / bc2) instead of sqrt(v) / sqrt(bc2) (reordered denominator) */
ORC_API void orc_adamw_mutant(float* p, const float* g, float* m, float* v, int64_t n,
                              double lr, double beta1, double beta2, double eps, double wd,
                              double step, int mutant) {
    double bc[2];
    orc_bias_corrections(beta1, beta2, step, bc);
    double step_size = lr / bc[0];
    if (mutant == 1) step_size = lr;
    const float decay = (float)(1.0 - lr * wd);
    const float w1 = (float)(1.0 - beta1);
    const float b2 = (float)beta2;
    const float w2 = mutant == 2 ? (float)beta2 : (float)(1.0 - beta2);
    const float bc2s = (float)bc[1];
    const float bc2 = (float)(1.0 - pow(beta2, step));
    const float epsf = (float)eps;
    const float nss = mutant == 4 ? (float)step_size : (float)(-step_size);
    for (int64_t i = 0; i < n; i++) {
        float gi = g[i];
        float pi = p[i];
        if (wd != 0.0 && mutant != 3) pi = pi * decay;
        float mi = m[i];
        if (mutant == 5) { float t = w1 * (gi - mi); mi = mi + t; }
        else mi = fmaf(w1, gi - mi, mi);
        float vi = v[i] * b2;
        vi = fmaf(w2 * gi, gi, vi);
        float d = mutant == 6 ? sqrtf(vi / bc2) : sqrtf(vi) / bc2s;
        d = d + epsf;
        float u = (nss * mi) / d;
        pi = pi + u;
        if (wd != 0.0 && mutant == 3) pi = pi * decay;
        p[i] = pi;
        m[i] = mi;
        v[i] = vi;
    }
}

/* ------------------------------------------------------------------------- */
/* a9: GradScaler.update                                                      */
/* ------------------------------------------------------------------------- */

/* torch/amp/grad_scaler.py:529-536 -> torch._amp_update_scale_.  The factor
 * products are formed in double and rounded to float once; growth is refused
 * when it would overflow; any nonzero found_inf (NaN included) backs off. */
ORC_API void orc_scaler_update(float* scale, int32_t* tracker, float found_inf,
                               double growth, double backoff, int32_t interval) {
    if (found_inf != 0.0f) {
        *scale = (float)((double)*scale * backoff);
        *tracker = 0;
    } else {
        int32_t ok = *tracker + 1;
        if (ok == interval) {
            float ns = (float)((double)*scale * growth);
            if (isfinite(ns)) *scale = ns;
            *tracker = 0;
        } else {
            *tracker = ok;
        }
    }
}

/* src/minigpt/optim.py:276-289 cosine_lr, restated for the pinning tests. */
ORC_API double orc_cosine_lr(int64_t step, double base_lr, double min_lr, int64_t warmup, int64_t max_steps) {
    if (warmup > 0 && step < warmup) return base_lr * (double)(step + 1) / (double)warmup;
    if (step >= max_steps) return min_lr;
    int64_t decay_steps = max_steps - warmup;
    if (decay_steps < 1) decay_steps = 1;
    double progress = (double)(step - warmup) / (double)decay_steps;
    if (progress < 0.0) progress = 0.0;
    if (progress > 1.0) progress = 1.0;
    double coeff = 0.5 * (1.0 + cos(M_PI * progress));
    return min_lr + coeff * (base_lr - min_lr);
}
