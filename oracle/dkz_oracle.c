/*
 * dkz_oracle.c -- CPU restatement of darknet-zig's CPU twins (the parity
 * authority for the MI355X tensor-op layer).
 *
 * TEST INFRASTRUCTURE ONLY. Loaded by tests/, __graft_entry__.smoke() and
 * bench.py's cpu_baseline leg, never by the product path.
 *
 * Float semantics of the Zig sources, restated here:
 *   - Zig's default float mode is strict: no contraction, no reassociation.
 *     This file is compiled with -ffp-contract=off and without -ffast-math, so
 *     every expression below rounds exactly where the Zig one does. Only axpy
 *     (blas.zig:21-24) runs under @setFloatMode(.optimized); on an FMA-capable
 *     x86-64 host LLVM contracts its y + alpha*x to one fused multiply-add, so
 *     it is written with fmaf here.
 *   - Zig float literals are comptime values coerced to f32 at the point of
 *     use, so 0.1 is 0.1f, 0.000001 is 1e-6f and 0.00001 is 1e-5f. A product
 *     of two literals is folded at comptime before the coercion (selu's
 *     1.0507 * 1.6732 becomes the single f32 constant 1.75803124f).
 *   - @exp and @log on f32 lower to the C library's expf/logf; @sqrt is the
 *     correctly rounded square root; @max/@min ignore a NaN operand like
 *     fmaxf/fminf; @rem is C's %.
 *
 * Pinning (what checks each function beyond restating it) is documented per
 * test in tests/test_oracle_*.py. std.math.pow's bit-level rounding (used by
 * variance_delta) and the binding of @exp/@log to the host libm cannot be
 * pinned without a Zig 0.16 toolchain; variance_delta's tolerance class
 * (1e-5 relative) covers the former.
 */
#include "dkz_oracle.h"

#include <float.h>
#include <math.h>
#include <string.h>

/* ------------------------------------------------------------------------ */
/* blas.zig:13-46                                                            */
/* ------------------------------------------------------------------------ */

/* blas.zig:13-15 */
void ref_fill(float *x, size_t n, float alpha) {
    for (size_t i = 0; i < n; ++i) x[i] = alpha;
}

/* blas.zig:17-19 */
void ref_copy(const float *src, float *dst, size_t n) { memcpy(dst, src, n * sizeof(float)); }

/* blas.zig:21-24 (@setFloatMode(.optimized): contracted to fma) */
void ref_axpy(float alpha, const float *x, float *y, size_t n) {
    for (size_t i = 0; i < n; ++i) y[i] = fmaf(alpha, x[i], y[i]);
}

/* blas.zig:26-29 */
void ref_scal(float alpha, float *x, size_t n) {
    for (size_t i = 0; i < n; ++i) x[i] *= alpha;
}

/* blas.zig:31-33 */
void ref_mul(const float *x, float *y, size_t n) {
    for (size_t i = 0; i < n; ++i) y[i] *= x[i];
}

/* blas.zig:44-46: std.math.clamp(v, -alpha, alpha) = @max(-alpha, @min(v, alpha)) */
void ref_constrain_array(float alpha, float *x, size_t n) {
    for (size_t i = 0; i < n; ++i) x[i] = fmaxf(-alpha, fminf(x[i], alpha));
}

/* ------------------------------------------------------------------------ */
/* bias / scale, blas.zig:53-100                                             */
/* ------------------------------------------------------------------------ */

/* blas.zig:53-61 */
void ref_add_bias(float *output, const float *biases, size_t batch, size_t filters, size_t spatial) {
    for (size_t b = 0; b < batch; ++b)
        for (size_t f = 0; f < filters; ++f) {
            float *row = output + (b * filters + f) * spatial;
            const float bias = biases[f];
            for (size_t s = 0; s < spatial; ++s) row[s] += bias;
        }
}

/* blas.zig:63-71 */
void ref_scale_bias(float *output, const float *scales, size_t batch, size_t filters, size_t spatial) {
    for (size_t b = 0; b < batch; ++b)
        for (size_t f = 0; f < filters; ++f) {
            float *row = output + (b * filters + f) * spatial;
            const float sc = scales[f];
            for (size_t s = 0; s < spatial; ++s) row[s] *= sc;
        }
}

/* blas.zig:73-82: one sequential sum per (b, f) row, added to the update in
 * batch order. */
void ref_backward_bias(float *bias_updates, const float *delta, size_t batch, size_t filters,
                       size_t spatial) {
    for (size_t b = 0; b < batch; ++b)
        for (size_t f = 0; f < filters; ++f) {
            const float *row = delta + (b * filters + f) * spatial;
            float sum = 0.0f;
            for (size_t s = 0; s < spatial; ++s) sum += row[s];
            bias_updates[f] += sum;
        }
}

/* blas.zig:84-100: one sequential sum per filter over (b, s) of dv*xv. */
void ref_backward_scale(const float *x_norm, const float *delta, size_t batch, size_t filters,
                        size_t spatial, float *scale_updates) {
    for (size_t f = 0; f < filters; ++f) {
        float sum = 0.0f;
        for (size_t b = 0; b < batch; ++b) {
            const size_t base = (b * filters + f) * spatial;
            for (size_t s = 0; s < spatial; ++s) sum += delta[base + s] * x_norm[base + s];
        }
        scale_updates[f] += sum;
    }
}

/* ------------------------------------------------------------------------ */
/* batch normalisation, blas.zig:106-204                                     */
/* ------------------------------------------------------------------------ */

/* blas.zig:106-116 */
void ref_mean(const float *x, size_t batch, size_t filters, size_t spatial, float *out) {
    const float scale_f = 1.0f / (float)(batch * spatial);
    for (size_t f = 0; f < filters; ++f) {
        float sum = 0.0f;
        for (size_t b = 0; b < batch; ++b) {
            const float *row = x + (b * filters + f) * spatial;
            for (size_t s = 0; s < spatial; ++s) sum += row[s];
        }
        out[f] = sum * scale_f;
    }
}

/* blas.zig:121-135 (unbiased: batch*spatial - 1) */
void ref_variance(const float *x, const float *mean, size_t batch, size_t filters, size_t spatial,
                  float *out) {
    const float scale_f = 1.0f / (float)(batch * spatial - 1);
    for (size_t f = 0; f < filters; ++f) {
        float sum = 0.0f;
        const float m = mean[f];
        for (size_t b = 0; b < batch; ++b) {
            const float *row = x + (b * filters + f) * spatial;
            for (size_t s = 0; s < spatial; ++s) {
                const float d = row[s] - m;
                sum += d * d;
            }
        }
        out[f] = sum * scale_f;
    }
}

/* blas.zig:137-146: reciprocal of (sqrt(v) + 1e-6), then a multiply. */
void ref_normalize(float *x, const float *mean, const float *variance, size_t batch, size_t filters,
                   size_t spatial) {
    for (size_t b = 0; b < batch; ++b)
        for (size_t f = 0; f < filters; ++f) {
            float *row = x + (b * filters + f) * spatial;
            const float m = mean[f];
            const float inv = 1.0f / (sqrtf(variance[f]) + 1e-6f);
            for (size_t s = 0; s < spatial; ++s) row[s] = (row[s] - m) * inv;
        }
}

/* blas.zig:148-157 */
void ref_mean_delta(const float *delta, const float *variance, size_t batch, size_t filters,
                    size_t spatial, float *out) {
    for (size_t f = 0; f < filters; ++f) {
        float sum = 0.0f;
        for (size_t b = 0; b < batch; ++b) {
            const float *row = delta + (b * filters + f) * spatial;
            for (size_t s = 0; s < spatial; ++s) sum += row[s];
        }
        out[f] = sum * (-1.0f / sqrtf(variance[f] + 1e-5f));
    }
}

/* blas.zig:159-178: sum * -0.5 * pow(v + 1e-5, -1.5), left to right. */
void ref_variance_delta(const float *x, const float *delta, const float *mean, const float *variance,
                        size_t batch, size_t filters, size_t spatial, float *out) {
    for (size_t f = 0; f < filters; ++f) {
        float sum = 0.0f;
        const float m = mean[f];
        for (size_t b = 0; b < batch; ++b) {
            const size_t base = (b * filters + f) * spatial;
            for (size_t s = 0; s < spatial; ++s) sum += delta[base + s] * (x[base + s] - m);
        }
        out[f] = (sum * -0.5f) * ref_pow_f32(variance[f] + 1e-5f, -1.5f);
    }
}

/* blas.zig:180-204: dv*inv + vd*2*(xv-m)/denom + md/denom, left to right. */
void ref_normalize_delta(const float *x, const float *mean, const float *variance,
                         const float *mean_delta, const float *variance_delta, size_t batch,
                         size_t filters, size_t spatial, float *delta) {
    const float denom = (float)(spatial * batch);
    for (size_t b = 0; b < batch; ++b)
        for (size_t f = 0; f < filters; ++f) {
            const size_t base = (b * filters + f) * spatial;
            const float inv = 1.0f / sqrtf(variance[f] + 1e-5f);
            const float vd = variance_delta[f];
            const float md = mean_delta[f];
            const float m = mean[f];
            for (size_t s = 0; s < spatial; ++s) {
                const float dv = delta[base + s];
                const float xv = x[base + s];
                delta[base + s] = (dv * inv + ((vd * 2.0f) * (xv - m)) / denom) + md / denom;
            }
        }
}

/* ------------------------------------------------------------------------ */
/* softmax and losses, blas.zig:213-282                                      */
/* ------------------------------------------------------------------------ */

float ref_expf(float x) { return expf(x); }

/* blas.zig:213-223 */
void ref_softmax_one(const float *input, size_t n, float temp, size_t stride, float *output) {
    float largest = -FLT_MAX;
    for (size_t i = 0; i < n; ++i) largest = fmaxf(largest, input[i * stride]);
    float sum = 0.0f;
    for (size_t i = 0; i < n; ++i) {
        const float e = expf(input[i * stride] / temp - largest / temp);
        sum += e;
        output[i * stride] = e;
    }
    for (size_t i = 0; i < n; ++i) output[i * stride] /= sum;
}

/* blas.zig:225-242 */
void ref_softmax(const float *input, size_t n, size_t batch, size_t batch_offset, size_t groups,
                 size_t group_offset, size_t stride, float temp, float *output) {
    for (size_t b = 0; b < batch; ++b)
        for (size_t g = 0; g < groups; ++g) {
            const size_t off = b * batch_offset + g * group_offset;
            ref_softmax_one(input + off, n, temp, stride, output + off);
        }
}

/* blas.zig:247-252 */
void ref_softmax_cross_entropy(const float *pred, const float *truth, float *delta, float *err,
                               size_t n) {
    for (size_t i = 0; i < n; ++i) {
        const float p = pred[i], t = truth[i];
        err[i] = (t != 0.0f) ? -logf(p) : 0.0f;
        delta[i] = t - p;
    }
}

/* blas.zig:254-260 */
void ref_l2(const float *pred, const float *truth, float *delta, float *err, size_t n) {
    for (size_t i = 0; i < n; ++i) {
        const float diff = truth[i] - pred[i];
        err[i] = diff * diff;
        delta[i] = diff;
    }
}

/* blas.zig:262-268 */
void ref_l1(const float *pred, const float *truth, float *delta, float *err, size_t n) {
    for (size_t i = 0; i < n; ++i) {
        const float diff = truth[i] - pred[i];
        err[i] = fabsf(diff);
        delta[i] = (diff > 0.0f) ? 1.0f : -1.0f;
    }
}

/* blas.zig:270-282 (the +1 for diff < 0 is the reference's own sign) */
void ref_smooth_l1(const float *pred, const float *truth, float *delta, float *err, size_t n) {
    for (size_t i = 0; i < n; ++i) {
        const float diff = truth[i] - pred[i];
        const float a = fabsf(diff);
        if (a < 1.0f) {
            err[i] = diff * diff;
            delta[i] = diff;
        } else {
            err[i] = 2.0f * a - 1.0f;
            delta[i] = (diff < 0.0f) ? 1.0f : -1.0f;
        }
    }
}

/* ------------------------------------------------------------------------ */
/* shortcut, blas.zig:290-322                                                */
/* ------------------------------------------------------------------------ */

void ref_shortcut(size_t batch, size_t w1, size_t h1, size_t c1, const float *add, size_t w2,
                  size_t h2, size_t c2, float s1, float s2, float *out) {
    size_t stride = w1 / w2;
    size_t sample = w2 / w1;
    if (stride < 1) stride = 1;
    if (sample < 1) sample = 1;
    const size_t minw = w1 < w2 ? w1 : w2;
    const size_t minh = h1 < h2 ? h1 : h2;
    const size_t minc = c1 < c2 ? c1 : c2;
    for (size_t b = 0; b < batch; ++b)
        for (size_t k = 0; k < minc; ++k)
            for (size_t j = 0; j < minh; ++j)
                for (size_t i = 0; i < minw; ++i) {
                    const size_t oi = i * sample + w2 * (j * sample + h2 * (k + c2 * b));
                    const size_t ai = i * stride + w1 * (j * stride + h1 * (k + c1 * b));
                    out[oi] = s1 * out[oi] + s2 * add[ai];
                }
}

/* ------------------------------------------------------------------------ */
/* activations.zig:58-143                                                    */
/* ------------------------------------------------------------------------ */

enum {
    A_LOGISTIC = 0, A_RELU, A_RELIE, A_LINEAR, A_RAMP, A_TANH, A_PLSE, A_LEAKY,
    A_ELU, A_LOGGY, A_STAIR, A_HARDTAN, A_LHTAN, A_SELU
};

/* activations.zig:58-81 */
float ref_activate(float x, int a) {
    switch (a) {
    case A_LINEAR: return x;
    case A_LOGISTIC: return 1.0f / (1.0f + expf(-x));
    case A_LOGGY: return 2.0f / (1.0f + expf(-x)) - 1.0f;
    case A_RELU: return (x > 0.0f) ? x : 0.0f;
    case A_ELU: return (x >= 0.0f) ? x : expf(x) - 1.0f;
    case A_SELU: return (x >= 0.0f) ? 1.0507f * x : 1.75803124f * (expf(x) - 1.0f);
    case A_RELIE: return (x > 0.0f) ? x : 0.01f * x;
    case A_RAMP: return ((x > 0.0f) ? x : 0.0f) + 0.1f * x;
    case A_LEAKY: return (x > 0.0f) ? x : 0.1f * x;
    case A_TANH: {
        const float e = expf(2.0f * x);
        return (e - 1.0f) / (e + 1.0f);
    }
    case A_PLSE:
        if (x < -4.0f) return 0.01f * (x + 4.0f);
        if (x > 4.0f) return 0.01f * (x - 4.0f) + 1.0f;
        return 0.125f * x + 0.5f;
    case A_STAIR: {
        /* @intFromFloat is illegal behaviour outside i64's range or on NaN. */
        const float n = floorf(x);
        const int64_t ni = (int64_t)n;
        return (ni % 2 == 0) ? floorf(x / 2.0f) : (x - n) + floorf(x / 2.0f);
    }
    case A_HARDTAN: return fmaxf(-1.0f, fminf(x, 1.0f));
    case A_LHTAN:
        if (x < 0.0f) return 0.001f * x;
        if (x > 1.0f) return 0.001f * (x - 1.0f) + 1.0f;
        return x;
    }
    return x;
}

/* activations.zig:85-104 */
float ref_gradient(float y, int a) {
    switch (a) {
    case A_LINEAR: return 1.0f;
    case A_LOGISTIC: return (1.0f - y) * y;
    case A_LOGGY: {
        const float t = (y + 1.0f) / 2.0f;
        return (2.0f * (1.0f - t)) * t;
    }
    case A_RELU: return (y > 0.0f) ? 1.0f : 0.0f;
    case A_ELU: return (y >= 0.0f) ? 1.0f : y + 1.0f;
    case A_SELU: return (y >= 0.0f) ? 1.0507f : y + 1.75803124f;
    case A_RELIE: return (y > 0.0f) ? 1.0f : 0.01f;
    case A_RAMP: return ((y > 0.0f) ? 1.0f : 0.0f) + 0.1f;
    case A_LEAKY: return (y > 0.0f) ? 1.0f : 0.1f;
    case A_TANH: return 1.0f - y * y;
    case A_PLSE: return (y < 0.0f || y > 1.0f) ? 0.01f : 0.125f;
    case A_STAIR: return (floorf(y) == y) ? 0.0f : 1.0f;
    case A_HARDTAN: return (y > -1.0f && y < 1.0f) ? 1.0f : 0.0f;
    case A_LHTAN: return (y > 0.0f && y < 1.0f) ? 1.0f : 0.001f;
    }
    return 1.0f;
}

/* activations.zig:107-125: linear leaves x untouched; the hoisted leaky, relu
 * and logistic loops compute exactly activate()'s expressions. */
void ref_activate_array(float *x, size_t n, int a) {
    if (a == A_LINEAR) return;
    for (size_t i = 0; i < n; ++i) x[i] = ref_activate(x[i], a);
}

/* activations.zig:127-143: delta *= gradient(y). */
void ref_gradient_array(const float *y, size_t n, int a, float *delta) {
    if (a == A_LINEAR) return;
    for (size_t i = 0; i < n; ++i) delta[i] *= ref_gradient(y[i], a);
}

/* ------------------------------------------------------------------------ */
/* pooling, layers/pooling.zig                                               */
/* ------------------------------------------------------------------------ */

/* pooling.zig:33-34 (makeMaxpool): the single `padding` is the total extra
 * extent. Requires in_dim + pad >= size. */
size_t ref_maxpool_out_dim(size_t in_dim, size_t size, size_t stride, size_t pad) {
    return (in_dim + pad - size) / stride + 1;
}

/* pooling.zig:59-93 */
void ref_forward_maxpool(size_t batch, size_t h, size_t w, size_t c, size_t size, size_t stride,
                         size_t pad, const float *input, float *output, int32_t *indexes) {
    const long off = -(long)(pad / 2);
    const size_t oh = ref_maxpool_out_dim(h, size, stride, pad);
    const size_t ow = ref_maxpool_out_dim(w, size, stride, pad);
    for (size_t b = 0; b < batch; ++b)
        for (size_t k = 0; k < c; ++k)
            for (size_t i = 0; i < oh; ++i)
                for (size_t j = 0; j < ow; ++j) {
                    const size_t out_index = j + ow * (i + oh * (k + c * b));
                    float mx = -FLT_MAX;
                    int32_t mi = -1;
                    for (size_t n = 0; n < size; ++n)
                        for (size_t m = 0; m < size; ++m) {
                            const long ch = off + (long)(i * stride + n);
                            const long cw = off + (long)(j * stride + m);
                            if (ch < 0 || ch >= (long)h) continue;
                            if (cw < 0 || cw >= (long)w) continue;
                            const size_t index = (size_t)cw + w * ((size_t)ch + h * (k + b * c));
                            const float val = input[index];
                            if (val > mx) {
                                mx = val;
                                mi = (int32_t)index;
                            }
                        }
                    output[out_index] = mx;
                    indexes[out_index] = mi;
                }
}

/* pooling.zig:95-103: scatter in ascending output order. */
void ref_backward_maxpool(size_t out_n, const int32_t *indexes, const float *delta,
                          float *prev_delta) {
    for (size_t i = 0; i < out_n; ++i) {
        const int32_t index = indexes[i];
        if (index < 0) continue;
        prev_delta[index] += delta[i];
    }
}

/* pooling.zig:146-158 */
void ref_forward_avgpool(size_t batch, size_t w, size_t h, size_t c, const float *input,
                         float *output) {
    const size_t spatial = h * w;
    const float denom = (float)spatial;
    for (size_t b = 0; b < batch; ++b)
        for (size_t k = 0; k < c; ++k) {
            const float *row = input + spatial * (k + b * c);
            float sum = 0.0f;
            for (size_t s = 0; s < spatial; ++s) sum += row[s];
            output[k + b * c] = sum / denom;
        }
}

/* pooling.zig:160-172 */
void ref_backward_avgpool(size_t batch, size_t w, size_t h, size_t c, const float *out_delta,
                          float *in_delta) {
    const size_t spatial = h * w;
    const float denom = (float)spatial;
    for (size_t b = 0; b < batch; ++b)
        for (size_t k = 0; k < c; ++k) {
            float *row = in_delta + spatial * (k + b * c);
            const float d = out_delta[k + b * c] / denom;
            for (size_t s = 0; s < spatial; ++s) row[s] += d;
        }
}

/* ------------------------------------------------------------------------ */
/* Zig 0.16 std.math.pow for f32 (lib/std/math/pow.zig; un-vendored        */
/* dependency of blas.zig:176). The integer-power loop follows the Go-derived */
/* algorithm of that file: x^y = exp(yf*log x) * x1^yi * 2^(xe*yi).          */
/* ------------------------------------------------------------------------ */

static int is_odd_integer(float y) {
    if (fabsf(y) >= 16777216.0f) return 0; /* every float this large is even */
    const float r = truncf(y);
    if (r != y) return 0;
    return ((int64_t)r & 1) != 0;
}

float ref_pow_f32(float x, float y) {
    if (y == 0.0f || x == 1.0f) return 1.0f;
    if (isnan(x) || isnan(y)) return NAN;
    if (y == 1.0f) return x;
    if (x == 0.0f) {
        if (y < 0.0f) return is_odd_integer(y) ? copysignf(INFINITY, x) : INFINITY;
        return is_odd_integer(y) ? x : 0.0f;
    }
    if (isinf(y)) {
        if (x == -1.0f) return 1.0f;
        if ((fabsf(x) < 1.0f) == (y > 0.0f)) return 0.0f;
        return INFINITY;
    }
    if (isinf(x)) {
        if (x < 0.0f) return ref_pow_f32(1.0f / x, -y);
        if (y < 0.0f) return 0.0f;
        if (y > 0.0f) return INFINITY;
    }
    if (y == 0.5f) return sqrtf(x);
    if (y == -0.5f) return 1.0f / sqrtf(x);

    float yi;
    float yf = modff(fabsf(y), &yi);
    if (yf != 0.0f && x < 0.0f) return NAN;
    if (yi >= 2147483648.0f) return expf(y * logf(x));

    float a1 = 1.0f;
    int ae = 0;
    if (yf != 0.0f) {
        if (yf > 0.5f) {
            yf -= 1.0f;
            yi += 1.0f;
        }
        a1 = expf(yf * logf(x));
    }
    int xe;
    float x1 = frexpf(x, &xe);
    for (int32_t i = (int32_t)yi; i != 0; i >>= 1) {
        const int overflow_shift = 8 + 1;
        if (xe < -(1 << overflow_shift) || (1 << overflow_shift) < xe) {
            ae += xe;
            break;
        }
        if ((i & 1) == 1) {
            a1 *= x1;
            ae += xe;
        }
        x1 *= x1;
        xe <<= 1;
        if (x1 < 0.5f) {
            x1 += x1;
            xe -= 1;
        }
    }
    if (y < 0.0f) {
        a1 = 1.0f / a1;
        ae = -ae;
    }
    return scalbnf(a1, ae);
}

/* ------------------------------------------------------------------------ */
/* The rest of gpu.zig's op surface: ops whose only definition in the       */
/* reference is the device kernel (no CPU twin), restated from it, and the  */
/* CPU halves of the layers that call them.                                  */
/* ------------------------------------------------------------------------ */

/* darknet_kernels.hip:150-153 (add_scalar_kernel, behind gpu.zig:503
 * addScalar; the cost layer's label smoothing, misc.zig:186-188). */
void ref_add_scalar(float alpha, float *x, size_t n) {
    for (size_t i = 0; i < n; ++i) x[i] += alpha;
}

/* darknet_kernels.hip:168-175: Chris Wellons' "lowbias32" integer hash (Hash
 * Prospector), xorshift-multiply with two odd constants. */
uint32_t ref_hash_u32(uint32_t x) {
    x ^= x >> 16;
    x *= 0x7feb352du;
    x ^= x >> 15;
    x *= 0x846ca68bu;
    x ^= x >> 16;
    return x;
}

/* darknet_kernels.hip:177-183 (rand_uniform_kernel, gpu.zig:511 randUniform):
 * element i = top 24 bits of hash(seed ^ hash(i)) times 2^-24, in [0, 1).
 * ref_rand_uniform_from writes elements first .. first+n-1 of that sequence
 * (a window of a large buffer); ref_rand_uniform is the window at 0. */
void ref_rand_uniform_from(float *x, size_t n, uint32_t seed, size_t first) {
    for (size_t i = 0; i < n; ++i) {
        const uint32_t h = ref_hash_u32(seed ^ ref_hash_u32((uint32_t)(first + i)));
        x[i] = (float)(h >> 8) * (1.0f / 16777216.0f);
    }
}

void ref_rand_uniform(float *x, size_t n, uint32_t seed) { ref_rand_uniform_from(x, n, seed, 0); }

/* layers/misc.zig:105-127 (forwardDropout's mask step given the uniform
 * draws, and backwardDropout): a draw below `prob` zeroes the element,
 * otherwise it is multiplied by `scale`. gpu.zig:769 / .hip:189-192 apply the
 * same rule on the device. */
void ref_dropout(float *x, size_t n, const float *rand, float prob, float scale) {
    for (size_t i = 0; i < n; ++i) {
        if (rand[i] < prob)
            x[i] = 0.0f;
        else
            x[i] *= scale;
    }
}

/* gpu.zig:804-830 adamUpdate: the twins' scal/axpy/mul steps in the wrapper's
 * order, then darknet_kernels.hip:588-595 (adam_kernel, no CPU twin):
 * mhat = m / (1 - b1^t), vhat = v / (1 - b2^t), w += rate*mhat/(sqrt(vhat)+eps),
 * and finally d = 0. The step count t reaches powf as a float. */
void ref_adam_update(float *w, float *d, float *m, float *v, float b1, float b2, float eps,
                     float decay, float rate, size_t n, size_t batch, size_t t) {
    ref_scal(b1, m, n);
    ref_scal(b2, v, n);
    ref_axpy(-decay * (float)batch, w, d, n);
    ref_axpy(1.0f - b1, d, m, n);
    ref_mul(d, d, n);
    ref_axpy(1.0f - b2, d, v, n);
    const float c1 = 1.0f - powf(b1, (float)(int)t);
    const float c2 = 1.0f - powf(b2, (float)(int)t);
    for (size_t i = 0; i < n; ++i) {
        const float mhat = m[i] / c1;
        const float vhat = v[i] / c2;
        w[i] = w[i] + rate * mhat / (sqrtf(vhat) + eps);
    }
    ref_fill(d, n, 0.0f);
}

/* ------------------------------------------------------------------------ */
/* im2col.zig: the convolution lowering                                      */
/* ------------------------------------------------------------------------ */

/* im2col.zig:9-11 */
size_t ref_conv_out_dim(size_t size, size_t ksize, size_t stride, size_t pad) {
    return (size + 2 * pad - ksize) / stride + 1;
}

/* im2col.zig:13-49: column row c = (c_im, h_offset, w_offset); taps that fall
 * in the padding are 0. */
void ref_im2col(const float *data_im, size_t channels, size_t height, size_t width, size_t ksize,
                size_t stride, size_t pad, float *data_col) {
    const size_t hc = ref_conv_out_dim(height, ksize, stride, pad);
    const size_t wc = ref_conv_out_dim(width, ksize, stride, pad);
    const size_t cc = channels * ksize * ksize;
    for (size_t c = 0; c < cc; ++c) {
        const size_t w_off = c % ksize;
        const size_t h_off = (c / ksize) % ksize;
        const size_t c_im = c / ksize / ksize;
        for (size_t h = 0; h < hc; ++h) {
            const long row = (long)(h_off + h * stride) - (long)pad;
            float *dst = data_col + (c * hc + h) * wc;
            if (row < 0 || row >= (long)height) {
                memset(dst, 0, wc * sizeof(float));
                continue;
            }
            const float *src = data_im + (c_im * height + (size_t)row) * width;
            for (size_t w = 0; w < wc; ++w) {
                const long col = (long)(w_off + w * stride) - (long)pad;
                dst[w] = (col >= 0 && col < (long)width) ? src[col] : 0.0f;
            }
        }
    }
}

/* im2col.zig:54-83: the adjoint, accumulated into data_im in column order. */
void ref_col2im(const float *data_col, size_t channels, size_t height, size_t width, size_t ksize,
                size_t stride, size_t pad, float *data_im) {
    const size_t hc = ref_conv_out_dim(height, ksize, stride, pad);
    const size_t wc = ref_conv_out_dim(width, ksize, stride, pad);
    const size_t cc = channels * ksize * ksize;
    for (size_t c = 0; c < cc; ++c) {
        const size_t w_off = c % ksize;
        const size_t h_off = (c / ksize) % ksize;
        const size_t c_im = c / ksize / ksize;
        for (size_t h = 0; h < hc; ++h) {
            const long row = (long)(h_off + h * stride) - (long)pad;
            if (row < 0 || row >= (long)height) continue;
            float *dst = data_im + (c_im * height + (size_t)row) * width;
            const float *src = data_col + (c * hc + h) * wc;
            for (size_t w = 0; w < wc; ++w) {
                const long col = (long)(w_off + w * stride) - (long)pad;
                if (col < 0 || col >= (long)width) continue;
                dst[col] += src[w];
            }
        }
    }
}

/* ------------------------------------------------------------------------ */
/* gemm.zig: C = alpha*op(A)*op(B) + beta*C, row-major                       */
/* ------------------------------------------------------------------------ */

/* gemm.zig:185-228 (gemmPanel, mr = 4 rows at once; the vector width only
 * groups columns, each column's sum runs over p in order) and gemm.zig:230-244
 * (gemmRow for the rows left over). The loops run under
 * @setFloatMode(.optimized), so LLVM contracts the multiply-adds to fma on an
 * FMA host and may regroup them: the accumulate steps are written with fmaf
 * here, and any summation order within fp32 rounding error is as valid. */
static void gemm_panel_rows(int ta, size_t i0, size_t rows, size_t n, size_t k, float alpha,
                            const float *a, size_t lda, const float *b, size_t ldb, float *c,
                            size_t ldc) {
    for (size_t q = 0; q < n; ++q) {
        float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
        for (size_t p = 0; p < k; ++p) {
            const float bv = b[p * ldb + q];
            for (size_t r = 0; r < rows; ++r) {
                const float s = ta ? a[p * lda + i0 + r] : a[(i0 + r) * lda + p];
                acc[r] = fmaf(s, bv, acc[r]);
            }
        }
        for (size_t r = 0; r < rows; ++r) c[(i0 + r) * ldc + q] = fmaf(alpha, acc[r], c[(i0 + r) * ldc + q]);
    }
}

static void gemm_row(int ta, size_t i, size_t n, size_t k, float alpha, const float *a, size_t lda,
                     const float *b, size_t ldb, float *c, size_t ldc) {
    for (size_t p = 0; p < k; ++p) {
        const float scale = alpha * (ta ? a[p * lda + i] : a[i * lda + p]);
        if (scale == 0.0f) continue;
        for (size_t q = 0; q < n; ++q) c[i * ldc + q] = fmaf(scale, b[p * ldb + q], c[i * ldc + q]);
    }
}

/* gemm.zig:47-141 (gemm, runJob: beta first -- 0 clears the row, anything but
 * 1 scales it -- then the variant), :249-278 (gemmNT / gemmTT: one dot
 * product per output element, c += alpha*sum). */
void ref_gemm(int ta, int tb, size_t m, size_t n, size_t k, float alpha, const float *a, size_t lda,
              const float *b, size_t ldb, float beta, float *c, size_t ldc) {
    if (m == 0 || n == 0) return;
    if (beta != 1.0f) {
        for (size_t i = 0; i < m; ++i) {
            float *row = c + i * ldc;
            if (beta == 0.0f)
                memset(row, 0, n * sizeof(float));
            else
                for (size_t q = 0; q < n; ++q) row[q] *= beta;
        }
    }
    if (!tb) {
        size_t i = 0;
        for (; i + 4 <= m; i += 4) gemm_panel_rows(ta, i, 4, n, k, alpha, a, lda, b, ldb, c, ldc);
        for (; i < m; ++i) gemm_row(ta, i, n, k, alpha, a, lda, b, ldb, c, ldc);
        return;
    }
    for (size_t i = 0; i < m; ++i)
        for (size_t q = 0; q < n; ++q) {
            float sum = 0.0f;
            for (size_t p = 0; p < k; ++p) {
                const float av = ta ? a[i + p * lda] : a[i * lda + p];
                sum = fmaf(av, b[q * ldb + p], sum);
            }
            c[i * ldc + q] = fmaf(alpha, sum, c[i * ldc + q]);
        }
}
