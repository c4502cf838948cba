/*
 * dkz_oracle.h -- CPU restatement of darknet-zig's CPU twins for the tensor-op
 * layer. TEST INFRASTRUCTURE ONLY: the parity checker for the HIP path and the
 * CPU baseline timed beside it. Only tests/, __graft_entry__.smoke() and
 * bench.py's cpu_baseline leg may load this library; the product path never
 * does.
 *
 * Each function restates one function of the reference (cited file:line),
 * keeping its loop order, its expression order and its f32 roundings. The
 * reference is Zig 0.16, which is not installed here, so the Zig sources could
 * not be compiled; see the pinning notes in the .c file.
 *
 * Sizes are size_t where the reference uses usize. Layout is NCHW.
 */
#ifndef DKZ_ORACLE_H
#define DKZ_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* blas.zig:13-46 */
void ref_fill(float *x, size_t n, float alpha);
void ref_copy(const float *src, float *dst, size_t n);
void ref_axpy(float alpha, const float *x, float *y, size_t n);
void ref_scal(float alpha, float *x, size_t n);
void ref_mul(const float *x, float *y, size_t n);
void ref_constrain_array(float alpha, float *x, size_t n);

/* blas.zig:53-100 */
void ref_add_bias(float *output, const float *biases, size_t batch, size_t filters, size_t spatial);
void ref_scale_bias(float *output, const float *scales, size_t batch, size_t filters, size_t spatial);
void ref_backward_bias(float *bias_updates, const float *delta, size_t batch, size_t filters,
                       size_t spatial);
void ref_backward_scale(const float *x_norm, const float *delta, size_t batch, size_t filters,
                        size_t spatial, float *scale_updates);

/* blas.zig:106-204 */
void ref_mean(const float *x, size_t batch, size_t filters, size_t spatial, float *out);
void ref_variance(const float *x, const float *mean, size_t batch, size_t filters, size_t spatial,
                  float *out);
void ref_normalize(float *x, const float *mean, const float *variance, size_t batch, size_t filters,
                   size_t spatial);
void ref_mean_delta(const float *delta, const float *variance, size_t batch, size_t filters,
                    size_t spatial, float *out);
void ref_variance_delta(const float *x, const float *delta, const float *mean, const float *variance,
                        size_t batch, size_t filters, size_t spatial, float *out);
void ref_normalize_delta(const float *x, const float *mean, const float *variance,
                         const float *mean_delta, const float *variance_delta, size_t batch,
                         size_t filters, size_t spatial, float *delta);

/* blas.zig:213-282 */
void ref_softmax_one(const float *input, size_t n, float temp, size_t stride, float *output);
void ref_softmax(const float *input, size_t n, size_t batch, size_t batch_offset, size_t groups,
                 size_t group_offset, size_t stride, float temp, float *output);
void ref_softmax_cross_entropy(const float *pred, const float *truth, float *delta, float *err,
                               size_t n);
void ref_l2(const float *pred, const float *truth, float *delta, float *err, size_t n);
void ref_l1(const float *pred, const float *truth, float *delta, float *err, size_t n);
void ref_smooth_l1(const float *pred, const float *truth, float *delta, float *err, size_t n);

/* blas.zig:290-322 */
void ref_shortcut(size_t batch, size_t w1, size_t h1, size_t c1, const float *add, size_t w2,
                  size_t h2, size_t c2, float s1, float s2, float *out);

/* activations.zig:58-143 */
float ref_activate(float x, int a);
float ref_gradient(float y, int a);
void ref_activate_array(float *x, size_t n, int a);
void ref_gradient_array(const float *y, size_t n, int a, float *delta);

/* layers/pooling.zig:33-34, 59-103, 146-172 */
size_t ref_maxpool_out_dim(size_t in_dim, size_t size, size_t stride, size_t pad);
void ref_forward_maxpool(size_t batch, size_t h, size_t w, size_t c, size_t size, size_t stride,
                         size_t pad, const float *input, float *output, int32_t *indexes);
void ref_backward_maxpool(size_t out_n, const int32_t *indexes, const float *delta,
                          float *prev_delta);
void ref_forward_avgpool(size_t batch, size_t w, size_t h, size_t c, const float *input,
                         float *output);
void ref_backward_avgpool(size_t batch, size_t w, size_t h, size_t c, const float *out_delta,
                          float *in_delta);

/* gpu.zig:503 addScalar, :511 randUniform, :769 dropout, :804-830 adamUpdate
 * (device kernels darknet_kernels.hip:150-153, 168-192, 588-595; the dropout
 * rule is also layers/misc.zig:105-127's CPU loop). */
void ref_add_scalar(float alpha, float *x, size_t n);
uint32_t ref_hash_u32(uint32_t x);
void ref_rand_uniform(float *x, size_t n, uint32_t seed);
void ref_rand_uniform_from(float *x, size_t n, uint32_t seed, size_t first);
void ref_dropout(float *x, size_t n, const float *rand, float prob, float scale);
void ref_adam_update(float *w, float *d, float *m, float *v, float b1, float b2, float eps,
                     float decay, float rate, size_t n, size_t batch, size_t t);

/* im2col.zig:9-83 */
size_t ref_conv_out_dim(size_t size, size_t ksize, size_t stride, size_t pad);
void ref_im2col(const float *data_im, size_t channels, size_t height, size_t width, size_t ksize,
                size_t stride, size_t pad, float *data_col);
void ref_col2im(const float *data_col, size_t channels, size_t height, size_t width, size_t ksize,
                size_t stride, size_t pad, float *data_im);

/* gemm.zig:47-278: C = alpha*op(A)*op(B) + beta*C, row-major, ta/tb select
 * the transposed operand layouts. */
void ref_gemm(int ta, int tb, size_t m, size_t n, size_t k, float alpha, const float *a, size_t lda,
              const float *b, size_t ldb, float beta, float *c, size_t ldc);

/* Zig 0.16 std.math.pow(f32, x, y), used by blas.zig:176. */
float ref_pow_f32(float x, float y);

/* The exp the twins bind @exp to (libm expf), exposed so tests can call it. */
float ref_expf(float x);

#ifdef __cplusplus
}
#endif

#endif /* DKZ_ORACLE_H */
