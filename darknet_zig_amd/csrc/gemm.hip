// gemm.hip -- C = alpha*op(A)*op(B) + beta*C, row-major (src/gpu.zig:671-719,
// CPU twin src/gemm.zig:47-278), on gfx950's fp32 matrix cores.
//
// A workgroup of four wave64s owns a BM x BN tile of C; each wave a
// (BM/2) x (BN/2) quarter of it, as (BM/64) x (BN/64) blocks of 32x32 that
// v_mfma_f32_32x32x2_f32 accumulates two k at a time (products exact, sums
// in fp32). K advances in steps of 16: every thread loads its share of the
// next A and B slabs from global memory into registers while the waves run
// the current slab's MFMAs out of LDS; the registers then go to the other
// LDS buffer, so each step needs one barrier.
//
// LDS holds both slabs k-major (As[p][i], Bs[p][j]) whatever the operands'
// layouts: a lane of an MFMA reads A(i0 + lane%32, kk + lane/32) and
// B(kk + lane/32, j0 + lane%32), 32 consecutive words per half-wave; rows are
// padded by 32 words so the two halves fall in different banks. Global loads
// walk each operand's contiguous dimension (k for A row-major, m for A
// transposed, likewise for B), zero-filling past m, n and k.
//
// The epilogue follows gemm.zig:121-131 then :180-184: beta == 0 clears C
// (NaN included), beta == 1 keeps it, anything else scales it; then
// C += alpha*acc. Results agree with the CPU twin within fp32 summation
// error (the twin's own order depends on its host's vector width).
//
// Workgroups take tiles in groups of 8 tile-rows, so that the tiles running
// at once share A and B panels, and neighbouring tile numbers are placed on
// one XCD (workgroups are dealt to the 8 XCDs round robin) so that they
// share its L2.
#include "dkz_device.hpp"
#include "dkz_internal.hpp"

namespace dkz {
namespace {

typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int kBK = 16;
constexpr int kGroupM = 8;
constexpr int kXcds = 8;

struct GemmArgs {
    const float *a;
    const float *b;
    float *c;
    uint32_t m, n, k, lda, ldb, ldc;
    float alpha, beta;
    uint32_t tiles_m, tiles_n;
};

template <int BM, int BN>
__device__ __forceinline__ void tile_of(uint32_t w, const GemmArgs &g, uint32_t &tm, uint32_t &tn) {
    const uint32_t total = g.tiles_m * g.tiles_n;
    uint32_t t = w;
    if (total % kXcds == 0) t = (w % kXcds) * (total / kXcds) + w / kXcds;
    const uint32_t per_group = kGroupM * g.tiles_n;
    const uint32_t first_m = (t / per_group) * kGroupM;
    const uint32_t gsize = g.tiles_m - first_m < (uint32_t)kGroupM ? g.tiles_m - first_m : (uint32_t)kGroupM;
    const uint32_t in_group = t % per_group;
    tm = first_m + in_group % gsize;
    tn = in_group / gsize;
}

template <int BM, int BN, bool TA, bool TB>
__global__ __launch_bounds__(kBlock) void gemm_mfma_kernel(GemmArgs g) {
    constexpr int SA = BM + 32, SB = BN + 32;  // LDS row strides in words
    constexpr int NA = BM * kBK / kBlock, NB = BN * kBK / kBlock;
    constexpr int WM = BM / 2, WN = BN / 2, TM = WM / 32, TN = WN / 32;
    __shared__ float As[2][kBK * SA];
    __shared__ float Bs[2][kBK * SB];

    uint32_t tm, tn;
    tile_of<BM, BN>(blockIdx.x, g, tm, tn);
    const uint32_t m0 = tm * BM, n0 = tn * BN;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm0 = (wave >> 1) * WM, wn0 = (wave & 1) * WN;
    const int half = lane >> 5, l32 = lane & 31;

    // This thread's slab coordinates: (ai[r], ap[r]) of A and (bp[r], bj[r]) of B.
    auto a_coord = [&](int r, int &i, int &p) {
        if constexpr (TA) { i = tid % BM; p = tid / BM + (kBlock / BM) * r; }
        else { p = tid % kBK; i = tid / kBK + (kBlock / kBK) * r; }
    };
    auto b_coord = [&](int r, int &p, int &j) {
        if constexpr (TB) { p = tid % kBK; j = tid / kBK + (kBlock / kBK) * r; }
        else { j = tid % BN; p = tid / BN + (kBlock / BN) * r; }
    };

    float ra[NA], rb[NB];
    auto load = [&](uint32_t k0) {
#pragma unroll
        for (int r = 0; r < NA; ++r) {
            int i, p;
            a_coord(r, i, p);
            const uint32_t gi = m0 + i, gp = k0 + p;
            ra[r] = (gi < g.m && gp < g.k) ? g.a[TA ? gp * g.lda + gi : gi * g.lda + gp] : 0.0f;
        }
#pragma unroll
        for (int r = 0; r < NB; ++r) {
            int p, j;
            b_coord(r, p, j);
            const uint32_t gp = k0 + p, gj = n0 + j;
            rb[r] = (gp < g.k && gj < g.n) ? g.b[TB ? gj * g.ldb + gp : gp * g.ldb + gj] : 0.0f;
        }
    };
    auto store = [&](int buf) {
#pragma unroll
        for (int r = 0; r < NA; ++r) {
            int i, p;
            a_coord(r, i, p);
            As[buf][p * SA + i] = ra[r];
        }
#pragma unroll
        for (int r = 0; r < NB; ++r) {
            int p, j;
            b_coord(r, p, j);
            Bs[buf][p * SB + j] = rb[r];
        }
    };

    f32x16 acc[TM][TN];
#pragma unroll
    for (int ti = 0; ti < TM; ++ti)
#pragma unroll
        for (int tj = 0; tj < TN; ++tj)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[ti][tj][r] = 0.0f;

    const uint32_t steps = (g.k + kBK - 1) / kBK;
    load(0);
    store(0);
    __syncthreads();
    for (uint32_t s = 0; s < steps; ++s) {
        const int cur = s & 1;
        if (s + 1 < steps) load((s + 1) * kBK);
        const float *as = As[cur] + half * SA + wm0 + l32;
        const float *bs = Bs[cur] + half * SB + wn0 + l32;
#pragma unroll
        for (int kk = 0; kk < kBK; kk += 2) {
            float af[TM], bf[TN];
#pragma unroll
            for (int ti = 0; ti < TM; ++ti) af[ti] = as[kk * SA + ti * 32];
#pragma unroll
            for (int tj = 0; tj < TN; ++tj) bf[tj] = bs[kk * SB + tj * 32];
#pragma unroll
            for (int ti = 0; ti < TM; ++ti)
#pragma unroll
                for (int tj = 0; tj < TN; ++tj)
                    acc[ti][tj] = __builtin_amdgcn_mfma_f32_32x32x2f32(af[ti], bf[tj], acc[ti][tj], 0, 0, 0);
        }
        if (s + 1 < steps) store(cur ^ 1);
        __syncthreads();
    }

    // acc[ti][tj][r] is C(row, col) of the wave's block (ti, tj) with
    // row = 8*(r/4) + 4*(lane/32) + r%4 and col = lane%32.
#pragma unroll
    for (int ti = 0; ti < TM; ++ti)
#pragma unroll
        for (int tj = 0; tj < TN; ++tj) {
            const uint32_t j = n0 + wn0 + tj * 32 + l32;
            if (j >= g.n) continue;
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const uint32_t i = m0 + wm0 + ti * 32 + (r >> 2) * 8 + half * 4 + (r & 3);
                if (i < g.m) {
                    float *cp = g.c + i * g.ldc + j;
                    float cv = 0.0f;
                    if (g.beta != 0.0f) cv = (g.beta == 1.0f) ? *cp : *cp * g.beta;
                    *cp = cv + g.alpha * acc[ti][tj][r];
                }
            }
        }
}

template <int BM, int BN>
int launch_gemm(bool ta, bool tb, GemmArgs g) {
    g.tiles_m = div_up(g.m, BM);
    g.tiles_n = div_up(g.n, BN);
    const uint64_t tiles = (uint64_t)g.tiles_m * g.tiles_n;
    DKZ_REQUIRE(tiles <= 0x7fffffffull);
    const dim3 grid((uint32_t)tiles), block(kBlock);
    if (!ta && !tb) return launch("gemm_nn", gemm_mfma_kernel<BM, BN, false, false>, grid, block, g);
    if (ta && !tb) return launch("gemm_tn", gemm_mfma_kernel<BM, BN, true, false>, grid, block, g);
    if (!ta && tb) return launch("gemm_nt", gemm_mfma_kernel<BM, BN, false, true>, grid, block, g);
    return launch("gemm_tt", gemm_mfma_kernel<BM, BN, true, true>, grid, block, g);
}

// Extent in elements of a rows x cols row-major view with leading dimension ld.
inline uint64_t extent(uint64_t rows, uint64_t cols, uint64_t ld) { return rows == 0 || cols == 0 ? 0 : (rows - 1) * ld + cols; }

}  // namespace
}  // namespace dkz

using namespace dkz;

extern "C" {

int dkz_gemm(int ta, int tb, int m, int n, int k, float alpha, const float *a, int lda, const float *b, int ldb,
             float beta, float *c, int ldc) {
    DKZ_REQUIRE(m >= 0 && n >= 0 && k >= 0 && lda >= 0 && ldb >= 0 && ldc >= 0);
    if (m == 0 || n == 0) return 0;  // gpu.zig:686
    DKZ_REQUIRE(c != nullptr && ldc >= n);
    DKZ_REQUIRE(extent(m, n, ldc) <= kMaxElems);
    if (k > 0) {
        DKZ_REQUIRE(a != nullptr && b != nullptr);
        DKZ_REQUIRE(lda >= (ta ? m : k) && ldb >= (tb ? k : n));
        DKZ_REQUIRE(extent(ta ? k : m, ta ? m : k, lda) <= kMaxElems);
        DKZ_REQUIRE(extent(tb ? n : k, tb ? k : n, ldb) <= kMaxElems);
    }
    GemmArgs g{a, b, c, (uint32_t)m, (uint32_t)n, (uint32_t)k, (uint32_t)lda, (uint32_t)ldb, (uint32_t)ldc,
               alpha, beta, 0, 0};
    // 128x128 tiles once they alone give every CU a workgroup; 64x64 below.
    const uint64_t big_tiles = (uint64_t)div_up(m, 128) * div_up(n, 128);
    if (big_tiles >= 256) return launch_gemm<128, 128>(ta != 0, tb != 0, g);
    return launch_gemm<64, 64>(ta != 0, tb != 0, g);
}

}  // extern "C"
