// GPU tests of the public primitive layer cuflash::kernels::* (matmul, online softmax, tile
// I/O), linked against build/libcuflash_attn.so. The cases restate the reference's
// tests/unit/test_matmul.cu, test_online_softmax.cu and test_tile_io.cu (same shapes, inputs,
// seeds and tolerances), plus every exported matmul shape against a CPU product. Prints one line
// per check that fails and a final "primitives: P passed, F failed"; exits 1 on any failure.
//
// Built by cuflash-attn_amd/build.py into build/test_primitives; run by
// tests/test_primitives_gpu.py on a GPU.

#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdio>
#include <cstring>
#include <random>
#include <string>
#include <vector>

#include "cuflash/kernels/matmul.cuh"
#include "cuflash/kernels/online_softmax.cuh"
#include "cuflash/kernels/tile_io.cuh"

using cuflash::FlashAttentionError;
namespace k = cuflash::kernels;

static int g_pass = 0, g_fail = 0;
static std::string g_case;

static void check(bool ok, const std::string& what) {
    if (ok) {
        ++g_pass;
    } else {
        ++g_fail;
        std::printf("FAIL [%s] %s\n", g_case.c_str(), what.c_str());
    }
}
static void check_near(float got, float want, float tol, const char* what, int idx) {
    const bool ok = std::fabs(got - want) <= tol;  // false for NaN
    if (!ok) {
        char buf[256];
        std::snprintf(buf, sizeof buf, "%s[%d]: got %.8g want %.8g (tol %g)", what, idx, got,
                      want, tol);
        check(false, buf);
    } else {
        ++g_pass;
    }
}
static void check_err(FlashAttentionError got, FlashAttentionError want, const char* what) {
    check(got == want, std::string(what) + ": code " + std::to_string(static_cast<int>(got)) +
                           " want " + std::to_string(static_cast<int>(want)));
}

// Device buffer with host copies in and out.
template <typename T>
struct Dev {
    T* p = nullptr;
    size_t n = 0;
    explicit Dev(size_t count) : n(count) {
        if (hipMalloc(&p, count * sizeof(T)) != hipSuccess) p = nullptr;
        if (p && hipMemset(p, 0, count * sizeof(T)) != hipSuccess) p = nullptr;
    }
    Dev(const std::vector<T>& h) : Dev(h.size()) { put(h); }
    ~Dev() {
        if (p) (void)hipFree(p);
    }
    void put(const std::vector<T>& h) {
        if (hipMemcpy(p, h.data(), n * sizeof(T), hipMemcpyHostToDevice) != hipSuccess)
            check(false, "hipMemcpy H2D");
    }
    std::vector<T> get() const {
        std::vector<T> h(n);
        if (hipDeviceSynchronize() != hipSuccess) check(false, "hipDeviceSynchronize");
        if (hipMemcpy(h.data(), p, n * sizeof(T), hipMemcpyDeviceToHost) != hipSuccess)
            check(false, "hipMemcpy D2H");
        return h;
    }
};

static std::vector<float> uniform(size_t n, unsigned seed, float lo, float hi) {
    std::mt19937 gen(seed);
    std::uniform_real_distribution<float> dist(lo, hi);
    std::vector<float> v(n);
    for (auto& x : v) x = dist(gen);
    return v;
}

// ------------------------------------------------------------------------------------------
// matmul (reference tests/unit/test_matmul.cu)
// ------------------------------------------------------------------------------------------
enum Op { ABt, AB, ABacc, AtB };

// CPU product in the reference test's order (test_matmul.cu:41-85).
static std::vector<float> cpu_mm(Op op, const std::vector<float>& A, const std::vector<float>& B,
                                 const std::vector<float>& C0, int M, int N, int K, float scale) {
    std::vector<float> C(M * N);
    for (int i = 0; i < M; ++i)
        for (int j = 0; j < N; ++j) {
            float s = 0.0f;
            for (int kk = 0; kk < K; ++kk) {
                const float a = op == AtB ? A[kk * M + i] : A[i * K + kk];
                const float b = op == ABt ? B[j * K + kk] : B[kk * N + j];
                s += a * b;
            }
            C[i * N + j] = op == ABacc ? C0[i * N + j] + s * scale : s * scale;
        }
    return C;
}

template <int M, int N, int K>
static FlashAttentionError gpu_mm(Op op, const float* A, const float* B, float* C, float scale,
                                  hipStream_t s) {
    switch (op) {
        case ABt: return k::matmul_ABt<M, N, K>(A, B, C, scale, s);
        case AB: return k::matmul_AB<M, N, K>(A, B, C, scale, s);
        case ABacc: return k::matmul_AB_acc<M, N, K>(A, B, C, scale, s);
        default: return k::matmul_AtB<M, N, K>(A, B, C, scale, s);
    }
}

// Random operands in [-1, 1] (seed 42 as in the reference), compared with the CPU product.
template <int M, int N, int K>
static void mm_case(Op op, hipStream_t s, float scale, float tol) {
    static const char* names[] = {"ABt", "AB", "AB_acc", "AtB"};
    g_case = std::string("matmul_") + names[op] + "<" + std::to_string(M) + "," +
             std::to_string(N) + "," + std::to_string(K) + ">";
    std::mt19937 gen(42);
    std::uniform_real_distribution<float> dist(-1.0f, 1.0f);
    std::vector<float> A(M * K), B(K * N), C0(M * N);
    for (auto& v : A) v = dist(gen);
    for (auto& v : B) v = dist(gen);
    for (auto& v : C0) v = dist(gen);
    const auto want = cpu_mm(op, A, B, C0, M, N, K, scale);
    Dev<float> dA(A), dB(B), dC(C0);
    check_err(gpu_mm<M, N, K>(op, dA.p, dB.p, dC.p, scale, s), FlashAttentionError::SUCCESS,
              "status");
    const auto got = dC.get();
    for (int i = 0; i < M * N; ++i) check_near(got[i], want[i], tol, "C", i);
}

template <int M, int N, int K>
static void mm_all_ops(hipStream_t s) {
    const float scale = 1.0f / std::sqrt(static_cast<float>(K));
    const float tol = K >= 128 ? 1e-3f : 1e-4f;  // the reference's tolerances by K
    for (Op op : {ABt, AB, ABacc, AtB}) mm_case<M, N, K>(op, s, scale, tol);
}

static void test_matmul(hipStream_t s) {
    // Every exported shape and product (reference matmul.cu:236-319).
    mm_all_ops<64, 64, 32>(s);
    mm_all_ops<32, 32, 32>(s);
    mm_all_ops<64, 64, 64>(s);
    mm_all_ops<32, 32, 128>(s);
    mm_all_ops<64, 64, 128>(s);
    mm_all_ops<32, 64, 32>(s);
    mm_all_ops<32, 64, 64>(s);
    mm_all_ops<64, 32, 64>(s);

    {  // ABt_HeadDim64 (test_matmul.cu:132-158): ones, scale 1/8 -> 8
        g_case = "ABt_HeadDim64";
        Dev<float> dA(std::vector<float>(64 * 64, 1.0f)), dB(std::vector<float>(64 * 64, 1.0f));
        Dev<float> dC(64 * 64);
        check_err(k::matmul_ABt<64, 64, 64>(dA.p, dB.p, dC.p, 0.125f, s),
                  FlashAttentionError::SUCCESS, "status");
        const auto c = dC.get();
        for (int i = 0; i < 64 * 64; ++i) check_near(c[i], 8.0f, 1e-4f, "C", i);
    }
    {  // AB_acc_Accumulates (test_matmul.cu:279-305): 10 + 32 = 42
        g_case = "AB_acc_Accumulates";
        Dev<float> dA(std::vector<float>(32 * 32, 1.0f)), dB(std::vector<float>(32 * 64, 1.0f));
        Dev<float> dC(std::vector<float>(32 * 64, 10.0f));
        check_err(k::matmul_AB_acc<32, 64, 32>(dA.p, dB.p, dC.p, 1.0f, s),
                  FlashAttentionError::SUCCESS, "status");
        const auto c = dC.get();
        for (int i = 0; i < 32 * 64; ++i) check_near(c[i], 42.0f, 1e-4f, "C", i);
    }
    {  // NullPointerReturnsError (test_matmul.cu:353-368)
        g_case = "matmul NullPointer";
        Dev<float> v(64 * 64);
        check_err(k::matmul_ABt<64, 64, 32>(nullptr, v.p, v.p, 1.0f, s),
                  FlashAttentionError::NULL_POINTER, "A null");
        check_err(k::matmul_ABt<64, 64, 32>(v.p, nullptr, v.p, 1.0f, s),
                  FlashAttentionError::NULL_POINTER, "B null");
        check_err(k::matmul_ABt<64, 64, 32>(v.p, v.p, nullptr, 1.0f, s),
                  FlashAttentionError::NULL_POINTER, "C null");
    }
    {  // ScaleFactorApplied and ABt_Linearity (test_matmul.cu:375-452)
        g_case = "matmul scale linearity";
        Dev<float> dA(uniform(64 * 32, 1, -1.0f, 1.0f)), dB(uniform(64 * 32, 2, -1.0f, 1.0f));
        Dev<float> c1(64 * 64), c2(64 * 64);
        std::mt19937 gen(11);
        std::uniform_real_distribution<float> sd(0.1f, 2.0f);
        for (int trial = 0; trial < 5; ++trial) {
            const float s1 = trial == 0 ? 1.0f : sd(gen);
            const float s2 = trial == 0 ? 0.5f : sd(gen);
            (void)k::matmul_ABt<64, 64, 32>(dA.p, dB.p, c1.p, s1, s);
            (void)k::matmul_ABt<64, 64, 32>(dA.p, dB.p, c2.p, s2, s);
            const auto h1 = c1.get(), h2 = c2.get();
            for (int i = 0; i < 64 * 64; ++i)
                check_near(h2[i], h1[i] * (s2 / s1), trial == 0 ? 1e-5f : 1e-3f, "C2", i);
        }
    }
}

// ------------------------------------------------------------------------------------------
// online softmax (reference tests/unit/test_online_softmax.cu)
// ------------------------------------------------------------------------------------------
static std::vector<float> cpu_softmax(const std::vector<float>& x, int rows, int cols,
                                      std::vector<float>* lse) {
    std::vector<float> y(x.size());
    if (lse) lse->assign(rows, 0.0f);
    for (int r = 0; r < rows; ++r) {
        double m = -INFINITY, sum = 0.0;
        for (int c = 0; c < cols; ++c) m = std::max(m, static_cast<double>(x[r * cols + c]));
        for (int c = 0; c < cols; ++c) sum += std::exp(x[r * cols + c] - m);
        for (int c = 0; c < cols; ++c)
            y[r * cols + c] = static_cast<float>(std::exp(x[r * cols + c] - m) / sum);
        if (lse) (*lse)[r] = static_cast<float>(m + std::log(sum));
    }
    return y;
}

static void softmax_case(const char* name, const std::vector<float>& x, int rows, int cols,
                         int block, float tol_y, float tol_lse, hipStream_t s) {
    g_case = name;
    std::vector<float> lse_want;
    const auto want = cpu_softmax(x, rows, cols, &lse_want);
    Dev<float> dx(x), dy(x.size()), dl(rows);
    check_err(k::online_softmax_forward(dx.p, dy.p, dl.p, rows, cols, block, s),
              FlashAttentionError::SUCCESS, "status");
    const auto y = dy.get(), l = dl.get();
    for (size_t i = 0; i < y.size(); ++i) {
        check(std::isfinite(y[i]), "finite output " + std::to_string(i));
        check_near(y[i], want[i], tol_y, "y", static_cast<int>(i));
    }
    for (int r = 0; r < rows; ++r) check_near(l[r], lse_want[r], tol_lse, "lse", r);
    for (int r = 0; r < rows; ++r) {
        double sum = 0.0;
        for (int c = 0; c < cols; ++c) sum += y[r * cols + c];
        check_near(static_cast<float>(sum), 1.0f, 1e-4f, "row sum", r);
    }
}

static void test_online_softmax(hipStream_t s) {
    softmax_case("Forward_Basic",
                 {1, 2, 3, 4, 5, 6, 7, 8, -1, 0, 1, 0, -1, 0, 1, 0, 0.1f, 0.2f, 0.3f, 0.4f, 0.5f,
                  0.6f, 0.7f, 0.8f, 10, 10, 10, 10, 10, 10, 10, 10},
                 4, 8, 4, 1e-5f, 1e-4f, s);
    softmax_case("Forward_LargeInput", uniform(64 * 128, 42, -5.0f, 5.0f), 64, 128, 32, 1e-4f,
                 1e-4f, s);
    softmax_case("Forward_MultiBlockCrossWarp", uniform(3 * 96, 7, -8.0f, 8.0f), 3, 96, 64, 1e-4f,
                 1e-4f, s);
    softmax_case("Forward_NumericalStability",
                 {1000.0f, 1001.0f, 1002.0f, 999.0f, -1000.0f, -999.0f, -1001.0f, -998.0f}, 2, 4, 2,
                 1e-4f, 1e-3f, s);
    softmax_case("OutputSumsToOne", uniform(16 * 64, 42, -10.0f, 10.0f), 16, 64, 16, 1e-4f,
                 1e-4f, s);
    softmax_case("Forward_LongRows_Block128", uniform(5 * 1000, 3, -20.0f, 20.0f), 5, 1000, 200,
                 1e-4f, 1e-4f, s);
    {  // Primitives_InitUpdateFinalize (test_online_softmax.cu:234-313)
        g_case = "Primitives_InitUpdateFinalize";
        const int rows = 4;
        const float s1 = std::exp(1.0f - 4) + std::exp(2.0f - 4) + std::exp(3.0f - 4) + 1.0f;
        const float s2 = std::exp(5.0f - 8) + std::exp(6.0f - 8) + std::exp(7.0f - 8) + 1.0f;
        Dev<float> m(rows), l(rows), lse(rows), nrm(rows);
        Dev<float> bm1(std::vector<float>(rows, 4.0f)), bs1(std::vector<float>(rows, s1));
        Dev<float> bm2(std::vector<float>(rows, 8.0f)), bs2(std::vector<float>(rows, s2));
        check_err(k::online_softmax_init(m.p, l.p, rows, s), FlashAttentionError::SUCCESS, "init");
        const auto m0 = m.get(), l0 = l.get();
        for (int r = 0; r < rows; ++r) {
            check(std::isinf(m0[r]) && m0[r] < 0, "init m = -inf");
            check(l0[r] == 0.0f, "init l = 0");
        }
        check_err(k::online_softmax_update(bm1.p, bs1.p, m.p, l.p, rows, s),
                  FlashAttentionError::SUCCESS, "update 1");
        check_err(k::online_softmax_update(bm2.p, bs2.p, m.p, l.p, rows, s),
                  FlashAttentionError::SUCCESS, "update 2");
        check_err(k::online_softmax_finalize(m.p, l.p, lse.p, nrm.p, rows, s),
                  FlashAttentionError::SUCCESS, "finalize");
        double sum = 0.0;
        for (int v = 1; v <= 8; ++v) sum += std::exp(v - 8.0);
        const auto hl = lse.get(), hn = nrm.get();
        for (int r = 0; r < rows; ++r) {
            check_near(hl[r], static_cast<float>(8.0 + std::log(sum)), 1e-4f, "lse", r);
            check_near(hn[r], static_cast<float>(1.0 / sum), 1e-5f, "normalizer", r);
        }
    }
    {  // NullPointer, InvalidDimension, FinalizeNullNormalizer (test_online_softmax.cu:316-357)
        g_case = "softmax errors";
        Dev<float> v(16);
        check_err(k::online_softmax_init(nullptr, v.p, 4, s), FlashAttentionError::NULL_POINTER,
                  "init null");
        check_err(k::online_softmax_forward(nullptr, v.p, v.p, 4, 4, 2, s),
                  FlashAttentionError::NULL_POINTER, "forward null");
        check_err(k::online_softmax_update(v.p, nullptr, v.p, v.p, 4, s),
                  FlashAttentionError::NULL_POINTER, "update null");
        check_err(k::online_softmax_finalize(v.p, v.p, v.p, nullptr, 4, s),
                  FlashAttentionError::NULL_POINTER, "finalize null normalizer");
        check_err(k::online_softmax_init(v.p, v.p, 0, s), FlashAttentionError::INVALID_DIMENSION,
                  "init rows 0");
        check_err(k::online_softmax_forward(v.p, v.p, v.p, 0, 4, 2, s),
                  FlashAttentionError::INVALID_DIMENSION, "forward rows 0");
        check_err(k::online_softmax_forward(v.p, v.p, v.p, 4, 0, 2, s),
                  FlashAttentionError::INVALID_DIMENSION, "forward cols 0");
        check_err(k::online_softmax_forward(v.p, v.p, v.p, 4, 4, 0, s),
                  FlashAttentionError::INVALID_DIMENSION, "forward block 0");
    }
}

// ------------------------------------------------------------------------------------------
// tile I/O (reference tests/unit/test_tile_io.cu)
// ------------------------------------------------------------------------------------------
static void test_tile_io(hipStream_t s) {
    {  // LoadTileFP32_64x64 (test_tile_io.cu:65-104): window (32, 32) of a 128 x 128 tensor
        g_case = "LoadTileFP32_64x64";
        const auto src = uniform(128 * 128, 42, -10.0f, 10.0f);
        Dev<float> dsrc(src), ddst(64 * 64);
        check_err(k::load_tile<64, 64>(dsrc.p, ddst.p, 32, 32, 128, 128, 128, s),
                  FlashAttentionError::SUCCESS, "status");
        const auto d = ddst.get();
        for (int r = 0; r < 64; ++r)
            for (int c = 0; c < 64; ++c)
                check(d[r * 64 + c] == src[(32 + r) * 128 + 32 + c], "exact copy");
    }
    {  // LoadTileFP16_64x64 (test_tile_io.cu:107-146)
        g_case = "LoadTileFP16_64x64";
        const auto f = uniform(128 * 64, 42, -1.0f, 1.0f);
        std::vector<__half> src(f.size());
        for (size_t i = 0; i < f.size(); ++i) src[i] = __float2half(f[i]);
        Dev<__half> dsrc(src);
        Dev<float> ddst(64 * 64);
        check_err(k::load_tile<64, 64>(dsrc.p, ddst.p, 0, 0, 128, 64, 64, s),
                  FlashAttentionError::SUCCESS, "status");
        const auto d = ddst.get();
        for (int i = 0; i < 64 * 64; ++i) check(d[i] == __half2float(src[i]), "exact widening");
    }
    {  // LoadTileBoundaryHandling (test_tile_io.cu:149-189)
        g_case = "LoadTileBoundaryHandling";
        Dev<float> dsrc(std::vector<float>(100 * 100, 1.0f));
        Dev<float> ddst(std::vector<float>(64 * 64, -7.0f));
        check_err(k::load_tile<64, 64>(dsrc.p, ddst.p, 64, 64, 100, 100, 100, s),
                  FlashAttentionError::SUCCESS, "status");
        const auto d = ddst.get();
        for (int r = 0; r < 64; ++r)
            for (int c = 0; c < 64; ++c)
                check(d[r * 64 + c] == ((r < 36 && c < 36) ? 1.0f : 0.0f), "fill");
    }
    {  // StoreTileFP32_64x64 (test_tile_io.cu:192-245): window (64, 64), rest untouched
        g_case = "StoreTileFP32_64x64";
        std::vector<float> tile(64 * 64);
        for (int i = 0; i < 64 * 64; ++i) tile[i] = static_cast<float>(i);
        Dev<float> dt(tile), dd(128 * 128);
        check_err(k::store_tile<64, 64>(dt.p, dd.p, 64, 64, 128, 128, 128, s),
                  FlashAttentionError::SUCCESS, "status");
        const auto d = dd.get();
        for (int r = 0; r < 128; ++r)
            for (int c = 0; c < 128; ++c) {
                const bool in = r >= 64 && c >= 64;
                check(d[r * 128 + c] == (in ? tile[(r - 64) * 64 + c - 64] : 0.0f), "store");
            }
    }
    {  // StoreTileFP16_32x128 (test_tile_io.cu:248-290): RNE rounding
        g_case = "StoreTileFP16_32x128";
        std::vector<float> tile(32 * 128);
        for (int i = 0; i < 32 * 128; ++i) tile[i] = static_cast<float>(i) / 100.0f;
        Dev<float> dt(tile);
        Dev<__half> dd(64 * 128);
        check_err(k::store_tile<32, 128>(dt.p, dd.p, 0, 0, 64, 128, 128, s),
                  FlashAttentionError::SUCCESS, "status");
        const auto d = dd.get();
        for (int i = 0; i < 32 * 128; ++i)
            check(__half2float(d[i]) == __half2float(__float2half(tile[i])), "RNE store");
        for (int i = 32 * 128; i < 64 * 128; ++i) check(__half2float(d[i]) == 0.0f, "untouched");
    }
    {  // StoreTile boundary: a window past the tensor writes only its in-tensor part
        g_case = "StoreTileBoundary_32x64";
        Dev<float> dt(std::vector<float>(32 * 64, 3.0f)), dd(50 * 70);
        check_err(k::store_tile<32, 64>(dt.p, dd.p, 40, 30, 50, 70, 70, s),
                  FlashAttentionError::SUCCESS, "status");
        const auto d = dd.get();
        for (int r = 0; r < 50; ++r)
            for (int c = 0; c < 70; ++c)
                check(d[r * 70 + c] == ((r >= 40 && c >= 30) ? 3.0f : 0.0f), "clipped store");
    }
    {  // RoundTripLoadStore (test_tile_io.cu:293-338): window (16, 16)
        g_case = "RoundTripLoadStore";
        const auto src = uniform(128 * 128, 123, -5.0f, 5.0f);
        Dev<float> ds(src), dd(128 * 128);
        check_err(k::load_store_tile_roundtrip<64, 64>(ds.p, dd.p, 16, 16, 128, 128, 128, s),
                  FlashAttentionError::SUCCESS, "status");
        const auto d = dd.get();
        for (int r = 0; r < 128; ++r)
            for (int c = 0; c < 128; ++c) {
                const bool in = r >= 16 && r < 80 && c >= 16 && c < 80;
                check(d[r * 128 + c] == (in ? src[r * 128 + c] : 0.0f), "roundtrip");
            }
    }
    {  // Every exported tile shape: load then store through a strided tensor
        g_case = "tile shapes";
        const auto src = uniform(200 * 160, 9, -3.0f, 3.0f);
        Dev<float> ds(src);
        auto run = [&](auto br, auto bc) {
            constexpr int BR = decltype(br)::value, BC = decltype(bc)::value;
            Dev<float> tile(BR * BC), out(200 * 160);
            check_err(k::load_tile<BR, BC>(ds.p, tile.p, 170, 100, 190, 150, 160, s),
                      FlashAttentionError::SUCCESS, "load");
            check_err(k::store_tile<BR, BC>(tile.p, out.p, 170, 100, 190, 150, 160, s),
                      FlashAttentionError::SUCCESS, "store");
            const auto o = out.get();
            for (int r = 0; r < 200; ++r)
                for (int c = 0; c < 160; ++c) {
                    const bool in = r >= 170 && r < std::min(190, 170 + BR) && c >= 100 &&
                                    c < std::min(150, 100 + BC);
                    check(o[r * 160 + c] == (in ? src[r * 160 + c] : 0.0f), "shape copy");
                }
        };
        run(std::integral_constant<int, 64>(), std::integral_constant<int, 64>());
        run(std::integral_constant<int, 64>(), std::integral_constant<int, 32>());
        run(std::integral_constant<int, 32>(), std::integral_constant<int, 32>());
        run(std::integral_constant<int, 32>(), std::integral_constant<int, 64>());
        run(std::integral_constant<int, 32>(), std::integral_constant<int, 128>());
        run(std::integral_constant<int, 64>(), std::integral_constant<int, 128>());
    }
    {  // NullPointerReturnsError, InvalidDimensionReturnsError (test_tile_io.cu:341-381)
        g_case = "tile errors";
        Dev<float> v(128 * 128), w(64 * 64);
        check_err(k::load_tile<64, 64>(static_cast<const float*>(nullptr), w.p, 0, 0, 128, 128,
                                       128, s),
                  FlashAttentionError::NULL_POINTER, "src null");
        check_err(k::load_tile<64, 64>(v.p, nullptr, 0, 0, 128, 128, 128, s),
                  FlashAttentionError::NULL_POINTER, "dst null");
        check_err(k::load_tile<64, 64>(v.p, w.p, -1, 0, 128, 128, 128, s),
                  FlashAttentionError::INVALID_DIMENSION, "row_start -1");
        check_err(k::load_tile<64, 64>(v.p, w.p, 128, 0, 128, 128, 128, s),
                  FlashAttentionError::INVALID_DIMENSION, "row_start = max_rows");
        check_err(k::load_tile<64, 64>(v.p, w.p, 0, 0, 0, 128, 128, s),
                  FlashAttentionError::INVALID_DIMENSION, "max_rows 0");
        check_err(k::store_tile<64, 64>(w.p, v.p, 0, 128, 128, 128, 128, s),
                  FlashAttentionError::INVALID_DIMENSION, "col_start = max_cols");
        check_err(k::store_tile<64, 64>(w.p, v.p, 0, 0, 128, 128, 0, s),
                  FlashAttentionError::INVALID_DIMENSION, "stride 0");
        check_err(k::load_store_tile_roundtrip<64, 64>(v.p, nullptr, 0, 0, 128, 128, 128, s),
                  FlashAttentionError::NULL_POINTER, "roundtrip dst null");
    }
}

int main(int argc, char** argv) {
    const std::string only = argc > 1 ? argv[1] : "";
    hipStream_t s;
    if (hipStreamCreate(&s) != hipSuccess) {
        std::printf("primitives: no HIP device\n");
        return 2;
    }
    if (only.empty() || only == "matmul") test_matmul(s);
    if (only.empty() || only == "softmax") test_online_softmax(s);
    if (only.empty() || only == "tile") test_tile_io(s);
    (void)hipStreamDestroy(s);
    std::printf("primitives: %d passed, %d failed\n", g_pass, g_fail);
    return g_fail == 0 ? 0 : 1;
}
