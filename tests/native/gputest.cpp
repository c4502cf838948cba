// gputest.cpp -- the CPU-vs-GPU consistency check of src/gputest.zig, written
// against the C++ host mirror of gpu.zig (darknet_zig_amd/host/dkz_gpu.hpp).
// TEST INFRASTRUCTURE: the CPU side is the oracle (oracle/dkz_oracle.h), the
// restatement of the Zig CPU twins.
//
// Every section and size of gputest.zig:86-480 is here, in its order, with
// its seed (20240921), its U(-1,1) inputs and its report line: max abs and
// max rel difference, ok when either is within 1e-3 (gputest.zig:27-52).
// Each check is also held to this library's own bar: bit-exact for
// elementwise, broadcast, copy and index results; for reductions and softmax
// an element within 1e-5 of the twin, or at least as close to an f64
// evaluation as the twin is; for gemm, Higham's fp32 bound against f64. A
// last section covers the ops gputest does not (add_scalar, rand_uniform,
// dropout, adam, scale_bias and the backward_scale / variance_delta /
// normalize_delta steps of the batch-norm backward pass).
//
// Usage: gputest [device]   -- prints one line per check, then
// "P/N checks passed." and a JSON summary line; exit status 1 on any failure.
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>
#include <vector>

#include "dkz_gpu.hpp"
#include "dkz_oracle.h"

namespace gpu = dkz::gpu;
using Vec = std::vector<float>;

namespace {

constexpr float kTolerance = 1e-3f;  // gputest.zig:29

int checks = 0, failures = 0;
std::vector<std::string> failed;

// splitmix64-seeded xoshiro256**: the harness's generator (gputest.zig uses
// Zig's DefaultPrng; only the distribution matters here).
struct Rng {
    uint64_t s[4];
    explicit Rng(uint64_t seed) {
        for (auto &w : s) {
            seed += 0x9e3779b97f4a7c15ull;
            uint64_t z = seed;
            z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
            z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
            w = z ^ (z >> 31);
        }
    }
    static uint64_t rotl(uint64_t x, int k) { return (x << k) | (x >> (64 - k)); }
    uint64_t next() {
        const uint64_t r = rotl(s[1] * 5, 7) * 9, t = s[1] << 17;
        s[2] ^= s[0];
        s[3] ^= s[1];
        s[1] ^= s[2];
        s[0] ^= s[3];
        s[2] ^= t;
        s[3] = rotl(s[3], 45);
        return r;
    }
    float uniform(float lo, float hi) { return lo + (float)(next() >> 40) * (1.0f / 16777216.0f) * (hi - lo); }
    size_t index(size_t n) { return (size_t)(next() % n); }
};

void randomFill(Rng &rng, Vec &x) {
    for (auto &v : x) v = rng.uniform(-1, 1);
}

uint32_t canon_bits(float f) {
    uint32_t u;
    std::memcpy(&u, &f, 4);
    return std::isnan(f) ? 0x7fc00000u : u;
}

enum class Bar { kBitExact, kR5, kBound };

// gputest.zig:33-52, plus the strict bar. For kR5, ref64 holds the f64
// evaluation; for kBound, ref64 the f64 value and bound the per-element bound.
void report(const char *name, const Vec &cpu, const Vec &back, Bar bar, const std::vector<double> *ref64 = nullptr,
            const std::vector<double> *bound = nullptr) {
    ++checks;
    float max_diff = 0, max_rel = 0;
    size_t strict_bad = 0;
    for (size_t i = 0; i < cpu.size(); ++i) {
        const float a = cpu[i], b = back[i];
        const float d = std::fabs(a - b);
        if (!(d <= max_diff) && !std::isnan(d)) max_diff = d;
        const float scale = std::fmax(std::fabs(a), std::fabs(b));
        if (scale > 1e-4f && d / scale > max_rel) max_rel = d / scale;
        if (std::isnan(a) != std::isnan(b)) max_diff = INFINITY;
        bool ok = true;
        switch (bar) {
            case Bar::kBitExact: ok = canon_bits(a) == canon_bits(b); break;
            case Bar::kR5: {
                const double g = b, c = a, r = (*ref64)[i];
                ok = (g == c) || std::fabs(g - c) <= 1e-5 * std::fabs(c) || std::fabs(g - r) <= std::fabs(c - r);
                break;
            }
            case Bar::kBound: ok = std::fabs((double)b - (*ref64)[i]) <= (*bound)[i]; break;
        }
        strict_bad += ok ? 0 : 1;
    }
    const bool ok = (max_diff <= kTolerance || max_rel <= kTolerance) && strict_bad == 0;
    if (!ok) {
        ++failures;
        failed.push_back(name);
    }
    const char *bar_name = bar == Bar::kBitExact ? "bit-exact" : bar == Bar::kR5 ? "1e-5/f64" : "fp32 bound";
    std::printf("%-28s %s  max abs diff %12.4e  max rel %12.4e  %s: %zu of %zu off\n", name, ok ? "ok  " : "FAIL",
                (double)max_diff, (double)max_rel, bar_name, strict_bad, cpu.size());
}

Vec pull(gpu::Buf b, size_t n) {
    Vec h(n);
    gpu::pull(b, h);
    return h;
}

// f64 sums of the per-channel terms, each term rounded to f32 as the twin
// rounds it (blas.zig:73-178): x, x*y (the product in f32), or (x-m)^2 (the
// difference and the square in f32).
std::vector<double> chan_sum64(const Vec &x, const Vec *y, size_t B, size_t F, size_t S, const Vec *mean) {
    std::vector<double> out(F, 0.0);
    for (size_t b = 0; b < B; ++b)
        for (size_t f = 0; f < F; ++f)
            for (size_t s = 0; s < S; ++s) {
                const size_t i = (b * F + f) * S + s;
                float v = x[i];
                if (mean) v = v - (*mean)[f];
                const float t = y ? v * (*y)[i] : (mean ? v * v : v);
                out[f] += (double)t;
            }
    return out;
}

// ---- gputest.zig:86-154 -----------------------------------------------------------

void elementwise(Rng &rng) {
    const size_t n = 4099;  // deliberately not a multiple of the block size
    Vec a(n), b(n);
    randomFill(rng, a);
    randomFill(rng, b);
    {
        Vec cpu = b;
        ref_axpy(2.5f, a.data(), cpu.data(), n);
        gpu::Buf da = gpu::make(a), db = gpu::make(b);
        gpu::axpy(n, 2.5f, da, db);
        report("axpy", cpu, pull(db, n), Bar::kBitExact);
        gpu::free(da);
        gpu::free(db);
    }
    {
        Vec cpu = a;
        ref_scal(0.3f, cpu.data(), n);
        gpu::Buf da = gpu::make(a);
        gpu::scal(n, 0.3f, da);
        report("scal", cpu, pull(da, n), Bar::kBitExact);
        gpu::free(da);
    }
    const struct {
        const char *name;
        int code;
    } acts[] = {{"activate leaky", DKZ_LEAKY}, {"activate relu", DKZ_RELU}, {"activate logistic", DKZ_LOGISTIC},
                {"activate elu", DKZ_ELU},     {"activate tanh", DKZ_TANH}};
    for (const auto &act : acts) {
        Vec cpu = a;
        ref_activate_array(cpu.data(), n, act.code);
        gpu::Buf da = gpu::make(a);
        gpu::activateArray(da, n, act.code);
        report(act.name, cpu, pull(da, n), Bar::kBitExact);
        gpu::free(da);
    }
    {
        Vec y = a;
        ref_activate_array(y.data(), n, DKZ_LEAKY);
        Vec cpu = b;
        ref_gradient_array(y.data(), n, DKZ_LEAKY, cpu.data());
        gpu::Buf dy = gpu::make(y), dd = gpu::make(b);
        gpu::gradientArray(dy, n, DKZ_LEAKY, dd);
        report("gradient leaky", cpu, pull(dd, n), Bar::kBitExact);
        gpu::free(dy);
        gpu::free(dd);
    }
}

// ---- gputest.zig:156-250 ----------------------------------------------------------

void biasAndNorm(Rng &rng) {
    const size_t batch = 4, filters = 17, spatial = 53, n = batch * filters * spatial;
    Vec x(n), delta(n), biases(filters);
    randomFill(rng, x);
    randomFill(rng, delta);
    randomFill(rng, biases);
    {
        Vec cpu = x;
        ref_add_bias(cpu.data(), biases.data(), batch, filters, spatial);
        gpu::Buf dx = gpu::make(x), dbias = gpu::make(biases);
        gpu::addBias(dx, dbias, batch, filters, spatial);
        report("add_bias", cpu, pull(dx, n), Bar::kBitExact);
        gpu::free(dx);
        gpu::free(dbias);
    }
    {
        Vec cpu(filters, 0.0f);
        ref_backward_bias(cpu.data(), delta.data(), batch, filters, spatial);
        const auto r64 = chan_sum64(delta, nullptr, batch, filters, spatial, nullptr);
        gpu::Buf ddelta = gpu::make(delta), dupd = gpu::alloc(filters);
        gpu::backwardBias(dupd, ddelta, batch, filters, spatial);
        report("backward_bias", cpu, pull(dupd, filters), Bar::kR5, &r64);
        gpu::free(ddelta);
        gpu::free(dupd);
    }
    // The batch-norm statistics, then the normalisation that consumes them.
    Vec mean_cpu(filters), var_cpu(filters);
    ref_mean(x.data(), batch, filters, spatial, mean_cpu.data());
    ref_variance(x.data(), mean_cpu.data(), batch, filters, spatial, var_cpu.data());
    const double count = (double)(batch * spatial);
    std::vector<double> mean64 = chan_sum64(x, nullptr, batch, filters, spatial, nullptr);
    for (auto &v : mean64) v /= count;
    std::vector<double> var64 = chan_sum64(x, nullptr, batch, filters, spatial, &mean_cpu);
    for (auto &v : var64) v /= count - 1;

    gpu::Buf dx = gpu::make(x), dmean = gpu::alloc(filters), dvar = gpu::alloc(filters);
    gpu::mean(dx, batch, filters, spatial, dmean);
    report("mean", mean_cpu, pull(dmean, filters), Bar::kR5, &mean64);
    // variance of the CPU mean, so the check isolates the variance op
    gpu::push(dmean, mean_cpu);
    gpu::variance(dx, dmean, batch, filters, spatial, dvar);
    report("variance", var_cpu, pull(dvar, filters), Bar::kR5, &var64);
    {
        Vec cpu = x;
        ref_normalize(cpu.data(), mean_cpu.data(), var_cpu.data(), batch, filters, spatial);
        gpu::push(dvar, var_cpu);
        gpu::normalize(dx, dmean, dvar, batch, filters, spatial);
        report("normalize", cpu, pull(dx, n), Bar::kBitExact);
    }
    {
        Vec cpu(filters);
        ref_mean_delta(delta.data(), var_cpu.data(), batch, filters, spatial, cpu.data());
        std::vector<double> r64 = chan_sum64(delta, nullptr, batch, filters, spatial, nullptr);
        for (size_t f = 0; f < filters; ++f) r64[f] *= -1.0 / std::sqrt((double)var_cpu[f] + 1e-5);
        gpu::Buf ddelta = gpu::make(delta), dout = gpu::alloc(filters);
        gpu::meanDelta(ddelta, dvar, batch, filters, spatial, dout);
        report("mean_delta", cpu, pull(dout, filters), Bar::kR5, &r64);
        gpu::free(ddelta);
        gpu::free(dout);
    }
    gpu::free(dx);
    gpu::free(dmean);
    gpu::free(dvar);
}

// ---- gputest.zig:252-300 ----------------------------------------------------------

void softmaxAndLoss(Rng &rng) {
    const size_t batch = 8, classes = 137, n = batch * classes;
    Vec x(n), truth(n, 0.0f);
    randomFill(rng, x);
    for (size_t b = 0; b < batch; ++b) truth[b * classes + rng.index(classes)] = 1.0f;
    Vec cpu(n);
    ref_softmax(x.data(), classes, batch, classes, 1, classes, 1, 1.0f, cpu.data());
    std::vector<double> p64(n);
    for (size_t b = 0; b < batch; ++b) {
        double mx = -INFINITY, sum = 0;
        for (size_t c = 0; c < classes; ++c) mx = std::fmax(mx, (double)x[b * classes + c]);
        for (size_t c = 0; c < classes; ++c) sum += std::exp((double)x[b * classes + c] - mx);
        for (size_t c = 0; c < classes; ++c) p64[b * classes + c] = std::exp((double)x[b * classes + c] - mx) / sum;
    }
    gpu::Buf dx = gpu::make(x), dout = gpu::alloc(n);
    gpu::softmax(dx, classes, batch, classes, 1, classes, 1, 1.0f, dout);
    report("softmax", cpu, pull(dout, n), Bar::kR5, &p64);
    {
        Vec delta_cpu(n), err_cpu(n);
        ref_softmax_cross_entropy(cpu.data(), truth.data(), delta_cpu.data(), err_cpu.data(), n);
        // isolate the op: both sides start from the CPU probabilities
        gpu::push(dout, cpu);
        gpu::Buf dtruth = gpu::make(truth), ddelta = gpu::alloc(n), derr = gpu::alloc(n);
        gpu::softmaxCrossEntropy(n, dout, dtruth, ddelta, derr);
        report("softmax_x_ent delta", delta_cpu, pull(ddelta, n), Bar::kBitExact);
        std::vector<double> e64(n);
        for (size_t i = 0; i < n; ++i) e64[i] = truth[i] != 0.0f ? -std::log((double)cpu[i]) : 0.0;
        report("softmax_x_ent loss", err_cpu, pull(derr, n), Bar::kR5, &e64);
        gpu::free(dtruth);
        gpu::free(ddelta);
        gpu::free(derr);
    }
    gpu::free(dx);
    gpu::free(dout);
}

// ---- gputest.zig:302-345 ----------------------------------------------------------

void convHelpers(Rng &rng) {
    const size_t c = 5, h = 13, w = 11, ksize = 3, stride = 2, pad = 1;
    const size_t hc = ref_conv_out_dim(h, ksize, stride, pad), wc = ref_conv_out_dim(w, ksize, stride, pad);
    const size_t col_n = c * ksize * ksize * hc * wc;
    Vec im(c * h * w);
    randomFill(rng, im);
    Vec cpu_col(col_n);
    ref_im2col(im.data(), c, h, w, ksize, stride, pad, cpu_col.data());
    gpu::Buf dim = gpu::make(im), dcol = gpu::alloc(col_n);
    gpu::im2col(dim, c, h, w, ksize, stride, pad, dcol);
    report("im2col", cpu_col, pull(dcol, col_n), Bar::kBitExact);
    {
        Vec cpu_im(c * h * w, 0.0f);
        ref_col2im(cpu_col.data(), c, h, w, ksize, stride, pad, cpu_im.data());
        gpu::Buf dim2 = gpu::alloc(c * h * w);
        gpu::col2im(dcol, c, h, w, ksize, stride, pad, dim2);
        report("col2im", cpu_im, pull(dim2, c * h * w), Bar::kBitExact);
        gpu::free(dim2);
    }
    gpu::free(dim);
    gpu::free(dcol);
}

// ---- gputest.zig:347-387 ----------------------------------------------------------

void gemmAll(Rng &rng) {
    const size_t m = 37, n = 29, k = 53;
    Vec a(m * k), b(k * n), c0(m * n);
    randomFill(rng, a);
    randomFill(rng, b);
    randomFill(rng, c0);
    // The same values in transposed storage for ta / tb.
    Vec at(k * m), bt(n * k);
    for (size_t i = 0; i < m; ++i)
        for (size_t p = 0; p < k; ++p) at[p * m + i] = a[i * k + p];
    for (size_t p = 0; p < k; ++p)
        for (size_t q = 0; q < n; ++q) bt[q * k + p] = b[p * n + q];
    std::vector<double> r64(m * n), bound(m * n);
    const double u = std::ldexp(1.0, -24), g = (k + 3) * u / (1 - (k + 3) * u);
    for (size_t i = 0; i < m; ++i)
        for (size_t q = 0; q < n; ++q) {
            double s = 0, sa = 0;
            for (size_t p = 0; p < k; ++p) {
                s += (double)a[i * k + p] * b[p * n + q];
                sa += std::fabs((double)a[i * k + p] * b[p * n + q]);
            }
            r64[i * n + q] = 1.5 * s + c0[i * n + q];
            bound[i * n + q] = g * (1.5 * sa + std::fabs((double)c0[i * n + q]));
        }
    const bool flags[4][2] = {{false, false}, {true, false}, {false, true}, {true, true}};
    for (const auto &fl : flags) {
        const bool ta = fl[0], tb = fl[1];
        const size_t lda = ta ? m : k, ldb = tb ? k : n;
        const Vec &ha = ta ? at : a, &hb = tb ? bt : b;
        Vec cpu = c0;
        ref_gemm(ta, tb, m, n, k, 1.5f, ha.data(), lda, hb.data(), ldb, 1.0f, cpu.data(), n);
        gpu::Buf da = gpu::make(ha), db = gpu::make(hb), dc = gpu::make(c0);
        gpu::gemm(ta, tb, m, n, k, 1.5f, da, lda, db, ldb, 1.0f, dc, n);
        const std::string name = std::string("gemm ") + (ta ? "T" : "N") + (tb ? "T" : "N");
        report(name.c_str(), cpu, pull(dc, m * n), Bar::kBound, &r64, &bound);
        gpu::free(da);
        gpu::free(db);
        gpu::free(dc);
    }
}

// ---- gputest.zig:389-451 ----------------------------------------------------------

void pooling(Rng &rng) {
    const size_t batch = 3, c = 6, h = 14, w = 14, size = 2, stride = 2, pad = size - 1;
    const size_t oh = ref_maxpool_out_dim(h, size, stride, pad), ow = ref_maxpool_out_dim(w, size, stride, pad);
    const size_t in_n = batch * c * h * w, out_n = batch * c * oh * ow;
    Vec input(in_n);
    randomFill(rng, input);
    Vec cpu_out(out_n);
    std::vector<int32_t> cpu_idx(out_n);
    ref_forward_maxpool(batch, h, w, c, size, stride, pad, input.data(), cpu_out.data(), cpu_idx.data());
    gpu::Buf dinput = gpu::make(input), dout = gpu::alloc(out_n), didx = gpu::allocInts(out_n);
    // pooling.zig:105-108 (forwardMaxpoolGpu)
    gpu::forwardMaxpool(out_n, h, w, c, stride, size, pad, dinput, dout, didx);
    report("maxpool forward", cpu_out, pull(dout, out_n), Bar::kBitExact);
    {
        std::vector<int32_t> back_idx(out_n);
        gpu::pullInts(didx, back_idx);
        Vec cidx(out_n), gidx(out_n);  // int32 indexes below 2^24: exact as floats
        for (size_t i = 0; i < out_n; ++i) {
            cidx[i] = (float)cpu_idx[i];
            gidx[i] = (float)back_idx[i];
        }
        report("maxpool indexes", cidx, gidx, Bar::kBitExact);
    }
    // Backward: seed the output delta, then compare what lands in the input.
    Vec delta(out_n);
    randomFill(rng, delta);
    Vec cpu_in_delta(in_n, 0.0f);
    ref_backward_maxpool(out_n, cpu_idx.data(), delta.data(), cpu_in_delta.data());
    gpu::Buf ddelta = gpu::make(delta), dindelta = gpu::alloc(in_n);
    // pooling.zig:110-114 (backwardMaxpoolGpu)
    gpu::backwardMaxpool(in_n, h, w, c, stride, size, pad, ddelta, dindelta, didx);
    report("maxpool backward", cpu_in_delta, pull(dindelta, in_n), Bar::kBitExact);

    Vec cpu_avg(batch * c);
    ref_forward_avgpool(batch, w, h, c, input.data(), cpu_avg.data());
    std::vector<double> avg64(batch * c, 0.0);
    for (size_t r = 0; r < batch * c; ++r) {
        for (size_t s = 0; s < h * w; ++s) avg64[r] += input[r * h * w + s];
        avg64[r] /= (double)(h * w);
    }
    gpu::Buf davg = gpu::alloc(batch * c);
    gpu::forwardAvgpool(batch * c, w, h, c, dinput, davg);  // pooling.zig:174-176
    report("avgpool forward", cpu_avg, pull(davg, batch * c), Bar::kR5, &avg64);
    for (gpu::Buf bb : {dinput, dout, didx, ddelta, dindelta, davg}) gpu::free(bb);
}

// ---- gputest.zig:453-480 ----------------------------------------------------------

void shortcutOp(Rng &rng) {
    const size_t batch = 2, w = 8, h = 8, c = 4, n = batch * w * h * c;
    Vec add(n), out(n);
    randomFill(rng, add);
    randomFill(rng, out);
    Vec cpu = out;
    ref_shortcut(batch, w, h, c, add.data(), w, h, c, 1, 1, cpu.data());
    gpu::Buf dadd = gpu::make(add), dout = gpu::make(out);
    gpu::shortcut(batch, w, h, c, dadd, w, h, c, 1, 1, dout);
    report("shortcut", cpu, pull(dout, n), Bar::kBitExact);
    gpu::free(dadd);
    gpu::free(dout);
}

// ---- beyond gputest.zig: the rest of the surface ----------------------------------

void restOfSurface(Rng &rng) {
    const size_t n = 4099;
    Vec a(n), b(n);
    randomFill(rng, a);
    randomFill(rng, b);
    {
        Vec cpu = a;
        ref_add_scalar(0.125f, cpu.data(), n);
        gpu::Buf da = gpu::make(a);
        gpu::addScalar(n, 0.125f, da);
        report("add_scalar", cpu, pull(da, n), Bar::kBitExact);
        gpu::free(da);
    }
    {
        // layers/misc.zig:128-141: randUniform, dropout forward and backward
        Vec r(n), x = a, d = b;
        ref_rand_uniform(r.data(), n, 0xC0FFEEu);
        ref_dropout(x.data(), n, r.data(), 0.3f, 1.0f / 0.7f);
        ref_dropout(d.data(), n, r.data(), 0.3f, 1.0f / 0.7f);
        gpu::Buf dr = gpu::alloc(n), dx = gpu::make(a), dd = gpu::make(b);
        gpu::randUniform(n, dr, 0xC0FFEEu);
        gpu::dropout(dx, n, dr, 0.3f, 1.0f / 0.7f);
        gpu::dropout(dd, n, dr, 0.3f, 1.0f / 0.7f);
        report("rand_uniform", r, pull(dr, n), Bar::kBitExact);
        report("dropout forward", x, pull(dx, n), Bar::kBitExact);
        report("dropout backward", d, pull(dd, n), Bar::kBitExact);
        for (gpu::Buf bb : {dr, dx, dd}) gpu::free(bb);
    }
    {
        Vec w = a, d = b, m(n, 0.0f), v(n, 0.0f);
        gpu::Buf dw = gpu::make(w), dd = gpu::alloc(n), dm = gpu::make(m), dv = gpu::make(v);
        for (size_t t = 1; t <= 3; ++t) {
            Vec dt = b;
            for (auto &e : dt) e *= 0.05f * (float)t;
            gpu::push(dd, dt);
            ref_adam_update(w.data(), dt.data(), m.data(), v.data(), 0.9f, 0.999f, 1e-7f, 0.0005f, 0.001f, n, 16,
                            t);
            gpu::adamUpdate(dw, dd, dm, dv, 0.9f, 0.999f, 1e-7f, 0.0005f, 0.001f, n, 16, t);
        }
        report("adam w", w, pull(dw, n), Bar::kBitExact);
        report("adam m", m, pull(dm, n), Bar::kBitExact);
        report("adam v", v, pull(dv, n), Bar::kBitExact);
        for (gpu::Buf bb : {dw, dd, dm, dv}) gpu::free(bb);
    }
    {
        // the batch-norm backward ops gputest leaves out, on CPU per-channel inputs
        const size_t B = 4, F = 17, S = 53, N = B * F * S;
        Vec x(N), xn(N), delta(N), scales(F);
        randomFill(rng, x);
        randomFill(rng, xn);
        randomFill(rng, delta);
        for (auto &s : scales) s = rng.uniform(0.5f, 1.5f);
        Vec mean(F), var(F);
        ref_mean(x.data(), B, F, S, mean.data());
        ref_variance(x.data(), mean.data(), B, F, S, var.data());
        gpu::Buf dx = gpu::make(x), dxn = gpu::make(xn), dd = gpu::make(delta), ds = gpu::make(scales);
        gpu::Buf dm = gpu::make(mean), dvv = gpu::make(var), out = gpu::alloc(F);
        {
            Vec cpu(F, 0.0f);
            ref_backward_scale(xn.data(), delta.data(), B, F, S, cpu.data());
            const auto r64 = chan_sum64(xn, &delta, B, F, S, nullptr);
            gpu::backwardScale(dxn, dd, B, F, S, out);
            report("backward_scale", cpu, pull(out, F), Bar::kR5, &r64);
        }
        {
            Vec cpu(F);
            ref_variance_delta(x.data(), delta.data(), mean.data(), var.data(), B, F, S, cpu.data());
            std::vector<double> r64(F, 0.0);
            for (size_t bb = 0; bb < B; ++bb)
                for (size_t f = 0; f < F; ++f)
                    for (size_t s = 0; s < S; ++s) {
                        const size_t i = (bb * F + f) * S + s;
                        r64[f] += (double)(delta[i] * (x[i] - mean[f]));  // f32 terms, blas.zig:174
                    }
            for (size_t f = 0; f < F; ++f) r64[f] *= -0.5 * std::pow((double)var[f] + 1e-5, -1.5);
            gpu::varianceDelta(dx, dd, dm, dvv, B, F, S, out);
            report("variance_delta", cpu, pull(out, F), Bar::kR5, &r64);
            // normalize_delta from the CPU per-channel deltas: bit-exact
            Vec md(F), vd = cpu, dcpu = delta;
            ref_mean_delta(delta.data(), var.data(), B, F, S, md.data());
            ref_normalize_delta(x.data(), mean.data(), var.data(), md.data(), vd.data(), B, F, S, dcpu.data());
            gpu::Buf dmd = gpu::make(md), dvd = gpu::make(vd);
            gpu::normalizeDelta(dx, dm, dvv, dmd, dvd, B, F, S, dd);
            report("normalize_delta", dcpu, pull(dd, N), Bar::kBitExact);
            gpu::free(dmd);
            gpu::free(dvd);
        }
        {
            Vec cpu = x;
            ref_scale_bias(cpu.data(), scales.data(), B, F, S);
            gpu::scaleBias(dx, ds, B, F, S);
            report("scale_bias", cpu, pull(dx, N), Bar::kBitExact);
        }
        for (gpu::Buf bb : {dx, dxn, dd, ds, dm, dvv, out}) gpu::free(bb);
    }
}

}  // namespace

int main(int argc, char **argv) {
    const int device = argc > 1 ? std::atoi(argv[1]) : 0;
    try {
        gpu::init(device);
        // gputest.zig:64-69: name the faulting kernel, not the next memcpy
        gpu::setSyncAfterLaunch(true);
        Rng rng(20240921);
        std::printf("\nComparing CPU and %s implementations on %s (tolerance %.0e):\n\n", gpu::backend_label,
                    gpu::deviceName().c_str(), (double)kTolerance);
        elementwise(rng);
        biasAndNorm(rng);
        softmaxAndLoss(rng);
        convHelpers(rng);
        gemmAll(rng);
        pooling(rng);
        shortcutOp(rng);
        restOfSurface(rng);
        gpu::setSyncAfterLaunch(false);
        gpu::deinit();
    } catch (const gpu::Error &e) {
        std::printf("\n%s\n", e.what());
        std::printf("{\"checks\": %d, \"passed\": %d, \"error\": true}\n", checks, checks - failures);
        return 2;
    }
    std::printf("\n%d/%d checks passed.\n", checks - failures, checks);
    std::printf("{\"checks\": %d, \"passed\": %d, \"failed\": [", checks, checks - failures);
    for (size_t i = 0; i < failed.size(); ++i) std::printf("%s\"%s\"", i ? ", " : "", failed[i].c_str());
    std::printf("]}\n");
    return failures == 0 ? 0 : 1;
}
