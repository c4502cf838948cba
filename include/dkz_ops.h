/*
 * dkz_ops.h -- C ABI of the MI355X (gfx950) tensor-op layer for darknet-zig.
 *
 * This header is the whole drop-in boundary. It replaces two things in the
 * reference (Eightscer/darknet_zig):
 *
 *   - the HIP backend glue src/hip/hip.zig:60-135 (device, memory, sync), and
 *   - the launch half of src/gpu.zig: the 37-kernel registry (gpu.zig:188-233),
 *     code-object loading (gpu.zig:240-257, 283-319), launchDims/launch1d/
 *     launchPerFilter (gpu.zig:427-477) and each op wrapper's argument
 *     marshalling (gpu.zig:483-800).
 *
 * Every op keeps the argument order and meaning of its gpu.zig wrapper: device
 * pointers where gpu.zig passes a Buf's .ptr, `int` where gpu.zig casts a usize
 * with ci() (gpu.zig:416-418), `float` scalars and the activation code as an
 * int (src/activations.zig:11-27). Kernels are private to the library; no
 * module, function or launch symbol is exported.
 *
 * Conventions shared by every entry point:
 *   - Return value: 0 on success, otherwise a hipError_t value (decode it with
 *     dkz_error_string). gpu.zig's must() turns a nonzero value into a panic
 *     (gpu.zig:51-55); callers that want that behaviour do the same.
 *   - A negative size or a null pointer where elements must be touched returns
 *     hipErrorInvalidValue (1) and launches nothing.
 *   - n == 0 / filters == 0 / batch == 0 is a silent no-op, as launch1d and
 *     launchPerFilter make it (gpu.zig:468, 475).
 *   - Work is issued, in call order, on the library's current stream (the null
 *     stream unless dkz_set_stream chose another), asynchronously to the host,
 *     as the reference issues everything on the null stream (hip.zig:134).
 *     dkz_copy_to_host blocks until earlier work on that stream is done.
 *   - With sync-after-launch on (dkz_set_sync_after_launch, or the environment
 *     variable DARKNET_GPU_SYNC / DARKNET_HIP_SYNC read by dkz_init) each op
 *     waits for its kernels and returns the fault, and dkz_last_error_context
 *     names the kernel (gpu.zig:173-183, 321-327, 456-464).
 *   - Layout is NCHW: element (b, f, s) of a [batch, filters, spatial] tensor is
 *     at ((b * filters) + f) * spatial + s (src/blas.zig:51).
 *   - Results follow the CPU twins in src/blas.zig, src/activations.zig and
 *     src/layers/pooling.zig: elementwise and broadcast ops bit-exact, the
 *     per-channel and per-row reductions and softmax within 1e-5 relative,
 *     maxpool indices bit-exact.
 *   - The library owns one scratch buffer per device (130.5 MiB), allocated
 *     and zeroed by dkz_init: the f64 partial sums of the split per-channel
 *     reductions (2 MiB), the partial tiles of a split-K gemm or convolution
 *     weight gradient (128 MiB) and 64-bit slots (512 KiB: one 256-byte
 *     line per channel's meeting slot or arrival counter, and one 128-byte
 *     posting line per workgroup of a one-launch batch-norm pass), through
 *     which a reduction's workgroups hand each other their partial sums.
 *     Ops never allocate, and leave the slots they use at zero. Reductions or
 *     gemms issued concurrently on two streams of one device share that
 *     buffer and race; issue them on one stream (dkz_set_stream).
 *   - dkz_batchnorm_forward and dkz_batchnorm_backward may run as one launch
 *     whose workgroups meet per channel. A wait there is bounded (about a
 *     second); if it runs out (the GPU did not hold all of the launch's
 *     workgroups at once, e.g. with other work on the device) the
 *     workgroup's results are NaN and it adds nothing to rolling_mean,
 *     rolling_variance, bias_updates or scale_updates. The next
 *     dkz_synchronize or dkz_copy_to_host -- or the op itself under
 *     sync-after-launch -- then returns hipErrorLaunchTimeOut (702), with the
 *     kernel named by dkz_last_error_context, as a kernel fault would surface
 *     in the reference (gpu.zig:51-55, 456-464).
 *   - The library is built with hidden visibility: it exports exactly the
 *     functions declared here.
 */
#ifndef DKZ_OPS_H
#define DKZ_OPS_H

#include <stddef.h>

#if defined(__GNUC__)
#pragma GCC visibility push(default)
#endif

#ifdef __cplusplus
extern "C" {
#endif

/* Activation codes: the enum values of src/activations.zig:11-27. */
enum dkz_activation {
    DKZ_LOGISTIC = 0,
    DKZ_RELU = 1,
    DKZ_RELIE = 2,
    DKZ_LINEAR = 3,
    DKZ_RAMP = 4,
    DKZ_TANH = 5,
    DKZ_PLSE = 6,
    DKZ_LEAKY = 7,
    DKZ_ELU = 8,
    DKZ_LOGGY = 9,
    DKZ_STAIR = 10,
    DKZ_HARDTAN = 11,
    DKZ_LHTAN = 12,
    DKZ_SELU = 13
};

/* ------------------------------------------------------------------------ */
/* Device and memory glue                                                     */
/* ------------------------------------------------------------------------ */

/* gpu.zig:259-347 init(): select `device`, read DARKNET_GPU_SYNC, allocate the
 * device's reduction scratch and make the occupancy lookups the batch-norm
 * passes need (so that a later graph capture of any op makes no HIP query
 * for the first time). Returns hipErrorInvalidDevice (101) when `device` is
 * out of range (gpu.zig:274-277 NoSuchDevice). */
int dkz_init(int device);

/* hip.zig:69-71 deviceCount. */
int dkz_device_count(int *count);

/* hip.zig:77-81 deviceName; writes at most len-1 bytes plus a NUL. */
int dkz_device_name(int device, char *buf, int len);

/* hip.zig:83-85 memInfo. */
int dkz_mem_info(size_t *free_bytes, size_t *total_bytes);

/* gpu.zig:362-369 alloc(): hipMalloc followed by zero fill. bytes == 0 gives
 * *ptr = NULL and success, as alloc(0) returns a null Buf. */
int dkz_malloc(void **ptr, size_t bytes);

/* gpu.zig:384-387 free(); NULL is a no-op. */
int dkz_free(void *ptr);

/* hip.zig:95-97 memsetZero. Ordered on the current stream. */
int dkz_memset_zero(void *ptr, size_t bytes);

/* gpu.zig:389-393 push() / hip.zig:99-101 copyToDevice. Blocking. */
int dkz_copy_to_device(void *dst, const void *src, size_t bytes);

/* gpu.zig:395-405 pull()/pullInts() / hip.zig:103-105 copyToHost. Blocking,
 * after all earlier work on the current stream. Also reports (and clears) a
 * batch-norm channel-meeting time-out: hipErrorLaunchTimeOut after the copy. */
int dkz_copy_to_host(void *dst, const void *src, size_t bytes);

/* gpu.zig:407-410 sync() / hip.zig:107-109 synchronize. Also reports (and
 * clears) a batch-norm channel-meeting time-out: hipErrorLaunchTimeOut. */
int dkz_synchronize(void);

/* hip.zig:60-62 errorString. */
const char *dkz_error_string(int err);

/* gpu.zig:181-183 setSyncAfterLaunch. */
void dkz_set_sync_after_launch(int on);
int dkz_get_sync_after_launch(void);

/* Name of the kernel (and launch shape) behind the last nonzero return on
 * this host thread, or "" -- the text of gpu.zig:445-462's panic messages. */
const char *dkz_last_error_context(void);

/* No counterpart in the reference, which always uses the null stream: choose
 * the hipStream_t (passed as void*) that later ops and copies are issued on.
 * NULL selects the null stream again. The choice is process-wide. Split
 * reductions and gemms use the device's one scratch (partials and
 * per-channel counters), so two streams running them at the same time on
 * one device race: switch streams only between such ops, not to overlap
 * them. */
int dkz_set_stream(void *stream);
void *dkz_get_stream(void);

/* ------------------------------------------------------------------------ */
/* Elementwise ops (gpu.zig:483-521; CPU twins blas.zig:13-46,              */
/* activations.zig:107-143)                                                  */
/* ------------------------------------------------------------------------ */

/* gpu.zig:483 fill(x, n, alpha): x[i] = alpha.            blas.zig:13 */
int dkz_fill(float *x, int n, float alpha);

/* gpu.zig:487 copy(n, x, y): y[i] = x[i].                 blas.zig:17 */
int dkz_copy(int n, const float *x, float *y);

/* gpu.zig:491 axpy(n, alpha, x, y): y[i] = fmaf(alpha, x[i], y[i]) -- one
 * rounding, as blas.zig:21-24 contracts under @setFloatMode(.optimized). */
int dkz_axpy(int n, float alpha, const float *x, float *y);

/* gpu.zig:495 scal(n, alpha, x): x[i] *= alpha.           blas.zig:26 */
int dkz_scal(int n, float alpha, float *x);

/* gpu.zig:499 mul(n, x, y): y[i] *= x[i].                 blas.zig:31 */
int dkz_mul(int n, const float *x, float *y);

/* gpu.zig:503 addScalar(n, alpha, x): x[i] += alpha (darknet_kernels.hip:150-153;
 * the cost layer's label smoothing, layers/misc.zig:186-188). */
int dkz_add_scalar(int n, float alpha, float *x);

/* gpu.zig:507 constrainArray(n, alpha, x): clamp to [-alpha, alpha]; NaN
 * becomes +alpha as std.math.clamp does (blas.zig:44-46). */
int dkz_constrain(int n, float alpha, float *x);

/* gpu.zig:511 randUniform(n, x, seed): x[i] = (hash(seed ^ hash(i)) >> 8) * 2^-24,
 * a counter-based draw in [0, 1) that depends on (seed, i) only; hash is
 * Wellons' lowbias32 (darknet_kernels.hip:168-183, the only definition: the
 * CPU path draws from its own generator, layers/misc.zig:107). */
int dkz_rand_uniform(int n, float *x, unsigned int seed);

/* gpu.zig:515 activateArray(x, n, a): x[i] = act(x[i]) (activations.zig:58-81,
 * 107-125). Exp-based activations use a bit-exact restatement of the host
 * libm expf. */
int dkz_activate_array(float *x, int n, int a);

/* gpu.zig:519 gradientArray(x, n, a, delta): delta[i] *= grad(x[i]), where x is
 * the activation's output (activations.zig:85-104, 127-143). */
int dkz_gradient_array(const float *x, int n, int a, float *delta);

/* ------------------------------------------------------------------------ */
/* Bias / scale broadcasts and their reductions (gpu.zig:527-555,           */
/* blas.zig:53-100)                                                          */
/* ------------------------------------------------------------------------ */

/* gpu.zig:527 addBias: output[b,f,s] += biases[f].         blas.zig:53 */
int dkz_add_bias(float *output, const float *biases, int batch, int filters, int spatial);

/* gpu.zig:533 scaleBias: output[b,f,s] *= scales[f].       blas.zig:63 */
int dkz_scale_bias(float *output, const float *scales, int batch, int filters, int spatial);

/* gpu.zig:539-549 backwardBias: bias_updates[f] += sum over b,s of delta.
 * spatial == 1 takes gpu.zig:540-543's per-filter path. blas.zig:73 */
int dkz_backward_bias(float *bias_updates, const float *delta, int batch, int filters, int spatial);

/* gpu.zig:551 backwardScale: scale_updates[f] += sum of delta*x_norm.
 * blas.zig:84-100 */
int dkz_backward_scale(const float *x_norm, const float *delta, int batch, int filters, int spatial,
                       float *scale_updates);

/* ------------------------------------------------------------------------ */
/* Batch normalisation (gpu.zig:561-608, blas.zig:106-204)                   */
/* ------------------------------------------------------------------------ */

/* gpu.zig:561 mean: out[f] = (sum of x) * (1/(batch*spatial)).   blas.zig:106 */
int dkz_mean(const float *x, int batch, int filters, int spatial, float *out);

/* gpu.zig:567 variance: out[f] = (sum of (x-m)^2) * (1/(batch*spatial-1)).
 * blas.zig:121-135 */
int dkz_variance(const float *x, const float *mean, int batch, int filters, int spatial, float *out);

/* gpu.zig:573 normalize: x = (x - m) * (1/(sqrt(v) + 1e-6)).  blas.zig:137-146 */
int dkz_normalize(float *x, const float *mean, const float *variance, int batch, int filters,
                  int spatial);

/* gpu.zig:580 meanDelta: out[f] = (sum of delta) * (-1/sqrt(v + 1e-5)).
 * blas.zig:148-157 */
int dkz_mean_delta(const float *delta, const float *variance, int batch, int filters, int spatial,
                   float *out);

/* gpu.zig:586 varianceDelta: out[f] = (sum of delta*(x-m)) * -0.5 * (v+1e-5)^-1.5.
 * blas.zig:159-178 */
int dkz_variance_delta(const float *x, const float *delta, const float *mean, const float *variance,
                       int batch, int filters, int spatial, float *out);

/* gpu.zig:592-608 normalizeDelta: delta = delta*inv + vd*2*(x-m)/N + md/N.
 * blas.zig:180-204 */
int dkz_normalize_delta(const float *x, const float *mean, const float *variance,
                        const float *mean_delta, const float *variance_delta, int batch, int filters,
                        int spatial, float *delta);

/* ------------------------------------------------------------------------ */
/* Softmax and losses (gpu.zig:614-645, blas.zig:213-282)                    */
/* ------------------------------------------------------------------------ */

/* gpu.zig:614-629 softmax: per (b, g) group at b*batch_offset + g*group_offset,
 * n elements `stride` apart; max, exp(x/T - max/T), sum, divide.
 * blas.zig:213-242 */
int dkz_softmax(const float *input, int n, int batch, int batch_offset, int groups, int group_offset,
                int stride, float temp, float *output);

/* No single gpu.zig counterpart: the forward step of the softmax layer,
 * layers/misc.zig:63-76 (forwardSoftmaxGpu), as one call --
 * softmax(input, inputs/groups, batch, inputs, groups, inputs/groups, 1, temp,
 * output), then, when truth is not NULL, softmaxCrossEntropy(batch*inputs,
 * output, truth, delta, loss). Groups longer than 32 run both as one pass;
 * results equal the two calls'. inputs % groups != 0 is hipErrorInvalidValue
 * (misc.zig:20 asserts it). */
int dkz_softmax_layer_forward(int batch, int inputs, int groups, float temp, const float *input,
                              const float *truth, float *output, float *delta, float *loss);

/* gpu.zig:631 softmaxCrossEntropy: err = t != 0 ? -log(p) : 0; delta = t - p.
 * blas.zig:247-252 */
int dkz_softmax_cross_entropy(int n, const float *pred, const float *truth, float *delta, float *err);

/* gpu.zig:635 l2 / 639 l1 / 643 smoothL1.                 blas.zig:254-282 */
int dkz_l2(int n, const float *pred, const float *truth, float *delta, float *err);
int dkz_l1(int n, const float *pred, const float *truth, float *delta, float *err);
int dkz_smooth_l1(int n, const float *pred, const float *truth, float *delta, float *err);

/* ------------------------------------------------------------------------ */
/* Pooling and shortcut (gpu.zig:725-800, pooling.zig:59-172,               */
/* blas.zig:290-322)                                                         */
/* ------------------------------------------------------------------------ */

/* gpu.zig:725-741 forwardMaxpool, called from pooling.zig:105-108 with
 * out_n = out_h*out_w*c*batch; out_w = (in_w + pad - size)/stride + 1.
 * Window offset -pad/2; first maximum under strict '>'; indexes holds the
 * absolute flat input index, -1 for a window with no valid tap.
 * pooling.zig:59-93 */
int dkz_forward_maxpool(int out_n, int in_h, int in_w, int in_c, int stride, int size, int pad,
                        const float *input, float *output, int *indexes);

/* gpu.zig:743-759 backwardMaxpool, called from pooling.zig:110-114 with
 * in_n = h*w*c*batch: prev_delta[indexes[o]] += delta[o], contributions to one
 * element added in ascending o. indexes must come from dkz_forward_maxpool
 * with the same geometry. pooling.zig:95-103 */
int dkz_backward_maxpool(int in_n, int in_h, int in_w, int in_c, int stride, int size, int pad,
                         const float *delta, float *prev_delta, const int *indexes);

/* gpu.zig:761 forwardAvgpool(n = c*batch, w, h, c): out[r] = (sum of the
 * row's w*h inputs) / (w*h).                              pooling.zig:146-158 */
int dkz_forward_avgpool(int n, int w, int h, int c, const float *input, float *output);

/* gpu.zig:765 backwardAvgpool(n = c*batch, w, h, c, in_delta, out_delta):
 * in_delta[r, s] += out_delta[r] / (w*h).                 pooling.zig:160-172 */
int dkz_backward_avgpool(int n, int w, int h, int c, float *in_delta, const float *out_delta);

/* gpu.zig:773-800 shortcut: out = s1*out + s2*add over the overlapping
 * region, with stride = w1/w2 and sample = w2/w1 (each at least 1) computed
 * here as gpu.zig:786-793 does. Two products, then a sum; no fma.
 * blas.zig:290-322 */
int dkz_shortcut(int batch, int w1, int h1, int c1, const float *add, int w2, int h2, int c2,
                 float s1, float s2, float *out);

/* ------------------------------------------------------------------------ */
/* Convolution lowering (gpu.zig:651-669, im2col.zig:13-83)                   */
/* ------------------------------------------------------------------------ */

/* gpu.zig:651 im2col(im, channels, height, width, ksize, stride, pad, col): col
 * is channels*ksize*ksize rows of height_col*width_col, height_col =
 * (height + 2*pad - ksize)/stride + 1; row (c*ksize + kh)*ksize + kw holds
 * im[c, h*stride - pad + kh, w*stride - pad + kw], 0 in the padding.
 * ksize > height + 2*pad (or width) or stride < 1 is hipErrorInvalidValue.
 * im2col.zig:13-49 */
int dkz_im2col(const float *im, int channels, int height, int width, int ksize, int stride, int pad,
               float *col);

/* gpu.zig:661 col2im(col, channels, height, width, ksize, stride, pad, im): the
 * adjoint, accumulated: every column entry is added to the image element
 * im2col took it from, an element's contributions in column order.
 * im2col.zig:54-83 */
int dkz_col2im(const float *col, int channels, int height, int width, int ksize, int stride, int pad,
               float *im);

/* gpu.zig:671-719 gemm(ta, tb, m, n, k, alpha, a, lda, b, ldb, beta, c, ldc):
 * C = alpha*op(A)*op(B) + beta*C, all row-major; op(A) is m x k (A is k x m
 * with leading dimension lda when ta != 0), op(B) is k x n. beta == 0 clears
 * C first (NaN included), beta != 1 scales it (gemm.zig:121-131). fp32
 * products and sums on the matrix cores: results agree with the CPU twin
 * within fp32 summation error. m == 0 or n == 0 does nothing (gpu.zig:686);
 * a leading dimension below the row length is hipErrorInvalidValue.
 * gemm.zig:47-278 */
int dkz_gemm(int ta, int tb, int m, int n, int k, float alpha, const float *a, int lda, const float *b,
             int ldb, float beta, float *c, int ldc);

/* The forward loop of a convolutional layer (layers/convolutional.zig:240-260)
 * in one call, beside the per-image im2col + gemm it replaces: for image i <
 * batch and group j < groups,
 *     output(i, j) += weights(j) x im2col(input(i, j))
 * with m = filters/groups, k = ksize^2 * channels/groups, n = out_h*out_w,
 * out_h = (height + 2*pad - ksize)/stride + 1 (convolutional.zig:21-27),
 * output(i, j) = output + (i*groups + j)*m*n, weights(j) = weights + j*m*k,
 * input(i, j) = input + (i*groups + j)*(channels/groups)*height*width. Like
 * the layer's gemm calls it adds to output (the layer zero-fills it first),
 * and for ksize == 1 it multiplies by the input itself read as a k x n
 * matrix, as the layer does. The im2col operand is gathered inside the
 * product: no workspace. channels and filters must be multiples of groups.
 * Results agree with the per-image calls within fp32 summation error. */
int dkz_convolution_forward(int batch, int groups, int channels, int height, int width, int filters, int ksize,
                            int stride, int pad, const float *weights, const float *input, float *output);

/* The weight-gradient half of a convolutional layer's backward loop
 * (layers/convolutional.zig:288-297, one gemm(false, true, ...) per image
 * into the shared weight_updates) in one call: for each group j,
 *     weight_updates(j) += sum over images i of delta(i, j) x im2col(input(i, j))^T
 * with m, n, k, the offsets and the ksize-1 reading of the input as in
 * dkz_convolution_forward, delta(i, j) = delta + (i*groups + j)*m*n and
 * weight_updates(j) = weight_updates + j*m*k. The images' contributions are
 * summed in a fixed order; results agree with the per-image calls within fp32
 * summation error. No workspace. */
int dkz_convolution_weight_gradient(int batch, int groups, int channels, int height, int width, int filters,
                                    int ksize, int stride, int pad, const float *delta, const float *input,
                                    float *weight_updates);

/* The data-gradient half of a convolutional layer's backward loop
 * (layers/convolutional.zig:299-305, per image gemm(true, false, ...) into the
 * workspace with beta 0 and col2im into the previous layer's delta) in one
 * call: with m, n, k and the offsets as in dkz_convolution_forward and
 * input_delta(i, j) = input_delta + (i*groups + j)*(channels/groups)*height*width,
 *     ksize == 1: input_delta(i, j) = weights(j)^T x delta(i, j), written as
 *                 a k x n matrix (the layer's beta-0 gemm straight into it);
 *     otherwise:  input_delta(i, j) += col2im(weights(j)^T x delta(i, j)).
 * Results agree with the per-image calls within fp32 summation error. Uses
 * the library's scratch (32 Mi floats) for the flipped weights; no
 * workspace. */
int dkz_convolution_data_gradient(int batch, int groups, int channels, int height, int width, int filters,
                                  int ksize, int stride, int pad, const float *weights, const float *delta,
                                  float *input_delta);

/* gpu.zig:769 dropout(input, size, rand, prob, scale): input[i] = rand[i] < prob ?
 * 0 : input[i] * scale, the rule of layers/misc.zig:105-127 (forward after
 * randUniform, and backward on the delta with the same draws). */
int dkz_dropout(float *input, int size, const float *rand, float prob, float scale);

/* gpu.zig:804-830 adamUpdate(w, d, m, v, b1, b2, eps, decay, rate, n, batch, t):
 * the wrapper's eight launches -- scal(b1, m), scal(b2, v),
 * axpy(-decay*batch, w, d), axpy(1-b1, d, m), mul(d, d), axpy(1-b2, d, v),
 * w += rate*mhat/(sqrt(vhat)+eps) with mhat = m/(1-b1^t), vhat = v/(1-b2^t)
 * (darknet_kernels.hip:588-595), fill(d, 0) -- as one pass over the four
 * vectors with the same per-element roundings. w, d, m and v must not
 * overlap (hipErrorInvalidValue otherwise); b^t is the host libm's powf. */
int dkz_adam_update(float *w, float *d, float *m, float *v, float b1, float b2, float eps, float decay,
                    float rate, int n, int batch, int t);

/* ---- fused batch-norm layer passes ------------------------------------------
 * Each replaces a sequence of the calls above that the layers issue; the
 * per-op entry points stay. Results equal the sequence's: every element
 * expression is the same op's, in the same order, given the same per-channel
 * values; the per-channel sums are the channel reductions' (within 1e-5 of
 * the CPU twin, or closer to the exact value). Shapes with spatial % 4 != 0,
 * empty tensors or tensors not 16-byte aligned run the per-op sequence. */

/* Forward of a batch-normalised layer and its activation: the sequence of
 * layers/batchnorm.zig:129-153 (forwardGpu) followed by
 * convolutional.zig:269 (activateArray(output, n, activation)), for a tensor
 * of batch*filters*spatial floats.
 *   input != output: output = input first (the standalone batchnorm layer,
 *   batchnorm.zig:133); input == output: in place (a convolutional layer).
 *   x = the input (batchnorm.zig:134).
 *   train: mean, variance of the input per channel (blas.zig:106-135);
 *     rolling_mean = rolling_mean*0.99 + 0.01*mean, likewise rolling_variance
 *     (scal, then axpy: batchnorm.zig:140-143);
 *     x_norm = (input - mean) * (1/(sqrt(variance) + 1e-6)) (blas.zig:137-146);
 *   not train: normalised with rolling_mean / rolling_variance; mean,
 *     variance and x_norm are not touched (may be NULL).
 *   output = act(x_norm * scales + biases)   (blas.zig:53-71, activations.zig)
 * The statistics are one pass over the input: f64 sums of (x - c) and
 * (x - c)^2 about the channel's first element c. */
int dkz_batchnorm_forward(int batch, int filters, int spatial, int activation, int train,
                          const float *input, float *output, float *x, float *x_norm, float *mean,
                          float *variance, float *rolling_mean, float *rolling_variance,
                          const float *scales, const float *biases);

/* Backward of a batch-normalised layer and its activation: convolutional.zig:280
 * (gradientArray(output, n, activation, delta)) followed by
 * layers/batchnorm.zig:155-174 (backwardGpu): backward_bias, backward_scale,
 * scale_bias(delta), mean_delta, variance_delta, normalize_delta. mean and
 * variance are the statistics the forward normalised with (the batch ones
 * when training, the rolling ones otherwise, batchnorm.zig:159-160).
 * bias_updates and scale_updates accumulate; mean_delta, variance_delta and
 * delta are overwritten. output may be NULL when activation is linear. */
int dkz_batchnorm_backward(int batch, int filters, int spatial, int activation, const float *output,
                           float *delta, const float *x, const float *x_norm, const float *mean,
                           const float *variance, const float *scales, float *bias_updates,
                           float *scale_updates, float *mean_delta, float *variance_delta);

/* No counterpart in the reference: dkz_batchnorm_backward for callers that
 * cannot allocate device memory (code under HIP graph capture, serving
 * loops, harnesses that forbid hipMalloc). Same arguments, kernels and
 * results, bit for bit; its scratch is a static device array of 2 MiB of
 * partial sums + 512 KiB of counter slots per GPU (held until the process
 * ends) instead of the library's allocated scratch, and it calls no
 * hipMalloc/hipFree. Limit: the ABI's 2^31-1 elements, beyond which it
 * returns hipErrorInvalidValue. Every call on one GPU shares that array:
 * calls that overlap on one GPU (two streams or host threads) race. */
int dkz_batchnorm_backward_noalloc(int batch, int filters, int spatial, int activation, const float *output,
                                   float *delta, const float *x, const float *x_norm, const float *mean,
                                   const float *variance, const float *scales, float *bias_updates,
                                   float *scale_updates, float *mean_delta, float *variance_delta);

#ifdef __cplusplus
}
#endif

#if defined(__GNUC__)
#pragma GCC visibility pop
#endif

#endif /* DKZ_OPS_H */
