// Host-code sanitizer run of libbrik's runtime (brik_runtime.cpp), built into this executable with
// AddressSanitizer and UndefinedBehaviorSanitizer (host code only: the kernels are the ordinary gfx950
// code object). It drives every C-ABI entry point through the host paths a caller reaches: argument
// validation and error codes without a device, then, on a GPU, contexts, copies, the pinned upload
// ring, matmuls on each path, plans (plain, fused, the linked GLU pair, a pre-staged one), graphs,
// fences, top-k, MoE, convolution, f16 weights, the encoders and the no-allocation entry point, with
// loose numeric checks (the parity tests hold the exact ones). Any sanitizer report aborts the run.
//
// usage: host_sanitize          (device checks run when a device is present)
//        host_sanitize nodev    (host checks only)
// Exit status 0 when every check passed.
#include "brik.h"

#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <random>
#include <vector>

extern "C" const char* __asan_default_options()
{
    // the HIP runtime keeps allocations until exit; the check here is for memory errors
    return "detect_leaks=0:verify_asan_link_order=0:abort_on_error=1";
}

namespace {

int fails = 0;
brik_ctx* ctx = nullptr;

#define CHECK(c, ...)                                                                     \
    do {                                                                                  \
        if (!(c)) {                                                                       \
            std::fprintf(stderr, "FAIL %s:%d: ", __FILE__, __LINE__);                     \
            std::fprintf(stderr, __VA_ARGS__);                                            \
            std::fputc('\n', stderr);                                                     \
            ++fails;                                                                      \
        }                                                                                 \
    } while (0)
#define OK(call)                                                                          \
    do {                                                                                  \
        const int rc_ = (call);                                                           \
        if (rc_ != BRIK_OK) {                                                             \
            std::fprintf(stderr, "FAIL %s:%d: %s -> %d (%s)\n", __FILE__, __LINE__, #call, rc_, \
                         ctx ? brik_last_error(ctx) : "");                                \
            ++fails;                                                                      \
        }                                                                                 \
    } while (0)

std::mt19937 rng(12345);

std::vector<float> uniform(size_t n, float lo = -1.f, float hi = 1.f)
{
    std::uniform_real_distribution<float> d(lo, hi);
    std::vector<float> v(n);
    for (auto& e : v) e = d(rng);
    return v;
}

// A device buffer freed at scope end.
struct Dev {
    void* p = nullptr;
    size_t n = 0;
    explicit Dev(size_t bytes) : n(bytes) { OK(brik_alloc(ctx, bytes ? bytes : 16, &p)); }
    ~Dev() { if (p) brik_free(ctx, p); }
    Dev(const Dev&) = delete;
    Dev& operator=(const Dev&) = delete;
    template <class T> T* as() const { return static_cast<T*>(p); }
    template <class T> T* at(size_t byte_off) const { return reinterpret_cast<T*>(static_cast<char*>(p) + byte_off); }
};

template <class T>
std::vector<T> download(const void* src, size_t count)
{
    std::vector<T> v(count);
    OK(brik_d2h(ctx, v.data(), src, count * sizeof(T)));
    return v;
}

// normwise relative difference ||a - b|| / ||b||
double rel(const std::vector<float>& a, const std::vector<double>& b)
{
    double num = 0, den = 0;
    for (size_t i = 0; i < b.size(); ++i) {
        num += (a[i] - b[i]) * (a[i] - b[i]);
        den += b[i] * b[i];
    }
    return std::sqrt(num / (den > 0 ? den : 1));
}

std::vector<double> ref_matmul(const std::vector<float>& x, const std::vector<float>& w, int M, int K, int N)
{
    std::vector<double> y((size_t)M * N);
    for (int m = 0; m < M; ++m)
        for (int n = 0; n < N; ++n) {
            double s = 0;
            for (int k = 0; k < K; ++k) s += (double)x[(size_t)m * K + k] * w[(size_t)n * K + k];
            y[(size_t)m * N + n] = s;
        }
    return y;
}

// q4 planes of an N x K matrix encoded on the device from uniform weights, with their dequantized
// values (the reference for the matmuls).
struct Q4 {
    int N, K;
    Dev nib, sc, mn;
    std::vector<float> deq;
    Q4(int n, int k) : N(n), K(k), nib((size_t)n * k / 2), sc((size_t)n * k / 16), mn((size_t)n * k / 16)
    {
        const size_t ne = (size_t)N * K;
        auto w = uniform(ne);
        Dev src(ne * 4), out(ne * 4);
        OK(brik_h2d(ctx, src.p, w.data(), ne * 4));
        OK(brik_quantize_q4(ctx, src.as<float>(), nib.as<uint8_t>(), sc.as<uint16_t>(), mn.as<uint16_t>(), ne));
        OK(brik_dequant_q4_f32(ctx, nib.as<uint8_t>(), sc.as<uint16_t>(), mn.as<uint16_t>(), out.as<float>(), ne));
        OK(brik_sync(ctx));
        deq = download<float>(out.p, ne);
    }
};

void host_checks()
{
    for (int code = -8; code <= 1; ++code) CHECK(brik_strerror(code) != nullptr, "strerror(%d)", code);
    CHECK(brik_last_error(nullptr) != nullptr, "last_error(null)");
    brik_ctx* c = nullptr;
    CHECK(brik_create(0, nullptr) == BRIK_EINVAL, "create(null out)");
    CHECK(brik_create(-1, &c) == BRIK_ENODEV && c == nullptr, "create(-1)");
    CHECK(brik_create(1 << 20, &c) == BRIK_ENODEV && c == nullptr, "create(huge)");
    brik_destroy(nullptr);
    int n = -1;
    CHECK(brik_device_count(nullptr) == BRIK_EINVAL, "device_count(null)");
    // every context entry point refuses a null context
    float f = 0;
    void* p = nullptr;
    char stage[32];
    CHECK(brik_alloc(nullptr, 16, &p) == BRIK_EINVAL, "alloc");
    CHECK(brik_free(nullptr, nullptr) == BRIK_EINVAL, "free");
    CHECK(brik_h2d(nullptr, &f, &f, 4) == BRIK_EINVAL, "h2d");
    CHECK(brik_h2d_async(nullptr, &f, &f, 4) == BRIK_EINVAL, "h2d_async");
    CHECK(brik_d2h(nullptr, &f, &f, 4) == BRIK_EINVAL, "d2h");
    CHECK(brik_d2d(nullptr, &f, &f, 4) == BRIK_EINVAL, "d2d");
    CHECK(brik_sync(nullptr) == BRIK_EINVAL, "sync");
    CHECK(brik_self_validate(nullptr, stage, sizeof stage) == BRIK_EINVAL, "self_validate");
    CHECK(brik_matmul_t_q4(nullptr, &f, nullptr, nullptr, nullptr, &f, 1, 32, 1) == BRIK_EINVAL, "matmul q4");
    CHECK(brik_matmul_t_q8(nullptr, &f, nullptr, nullptr, &f, 1, 32, 1) == BRIK_EINVAL, "matmul q8");
    CHECK(brik_matmul_t_q3(nullptr, &f, nullptr, nullptr, nullptr, nullptr, &f, 1, 32, 1) == BRIK_EINVAL, "q3");
    CHECK(brik_matmul_t_q4_noalloc(nullptr, &f, nullptr, nullptr, nullptr, &f, 1, 32, 1) == BRIK_EINVAL, "noalloc");
    brik_gemv_plan* plan = nullptr;
    CHECK(brik_gemv_plan_create(nullptr, BRIK_FMT_Q4, nullptr, 0, &plan) == BRIK_EINVAL, "plan_create");
    CHECK(brik_gemv_plan_run(nullptr, nullptr) == BRIK_EINVAL, "plan_run");
    brik_gemv_plan_destroy(nullptr, nullptr);
    brik_graph* g = nullptr;
    CHECK(brik_graph_begin(nullptr) == BRIK_EINVAL, "graph_begin");
    CHECK(brik_graph_end(nullptr, &g) == BRIK_EINVAL, "graph_end");
    brik_graph_destroy(nullptr, nullptr);
    brik_fence* fe = nullptr;
    CHECK(brik_fence_record(nullptr, &fe) == BRIK_EINVAL, "fence_record");
    brik_fence_destroy(nullptr);
    CHECK(brik_set_option(nullptr, BRIK_OPT_PATH, 0) == BRIK_EINVAL, "set_option");
    CHECK(brik_timer_begin(nullptr) == BRIK_EINVAL, "timer_begin");
    CHECK(brik_timer_end(nullptr, &f) == BRIK_EINVAL, "timer_end");
    (void)n;
}

void copies()
{
    const size_t n = 1 << 20;
    auto h = uniform(n / 4);
    Dev a(n), b(n);
    OK(brik_h2d(ctx, a.p, h.data(), n));
    OK(brik_d2d(ctx, b.p, a.p, n));
    auto back = download<float>(b.p, n / 4);
    CHECK(std::memcmp(back.data(), h.data(), n) == 0, "h2d / d2d / d2h round trip");
    OK(brik_h2d(ctx, a.p, h.data(), 0));

    // the pinned upload ring: the bytes are taken at the call (the host buffer is overwritten right
    // after each call), uploads wrap the ring several times, odd sizes and offsets, one upload past
    // the ring's direct limit (the synchronous fallback)
    const size_t dev_bytes = 48u << 20;
    Dev d(dev_bytes);
    std::vector<unsigned char> expect(dev_bytes, 0), host(24u << 20);
    OK(brik_h2d(ctx, d.p, expect.data(), dev_bytes));
    size_t off = 0;
    const size_t sizes[] = {3u << 20, 1, 4097, 5u << 20, 7u << 20, 13, 2u << 20, 20u << 20, 0, 9u << 20};
    for (int rep = 0; rep < 4; ++rep)
        for (size_t s : sizes) {
            if (off + s > dev_bytes) off = (off * 7 + 3) % 4096;
            for (size_t i = 0; i < s; ++i) host[i] = (unsigned char)(rng() & 0xff);
            std::memcpy(expect.data() + off, host.data(), s);
            OK(brik_h2d_async(ctx, d.at<unsigned char>(off), host.data(), s));
            std::memset(host.data(), 0xA5, s);    // the upload must already hold its own copy
            off += s + 5;
        }
    OK(brik_sync(ctx));
    auto got = download<unsigned char>(d.p, dev_bytes);
    CHECK(got == expect, "h2d_async contents after wrapping the staging ring");
}

void matmuls()
{
    const int K = 512, N = 256;
    Q4 w(N, K);
    for (int M : {1, 3, 8, 24, 64, 200}) {
        auto x = uniform((size_t)M * K);
        Dev dx((size_t)M * K * 4), dy((size_t)M * N * 4), dz((size_t)M * N * 4);
        OK(brik_h2d(ctx, dx.p, x.data(), x.size() * 4));
        OK(brik_matmul_t_q4(ctx, dx.as<float>(), w.nib.as<uint8_t>(), w.sc.as<uint16_t>(), w.mn.as<uint16_t>(),
                            dy.as<float>(), M, K, N));
        const int path = brik_last_path(ctx);
        CHECK(path >= BRIK_PATH_GEMV && path <= BRIK_PATH_SPLITK, "M=%d path %d", M, path);
        OK(brik_matmul_t_q4_noalloc(ctx, dx.as<float>(), w.nib.as<uint8_t>(), w.sc.as<uint16_t>(),
                                    w.mn.as<uint16_t>(), dz.as<float>(), M, K, N));
        OK(brik_sync(ctx));
        auto y = download<float>(dy.p, (size_t)M * N), z = download<float>(dz.p, (size_t)M * N);
        const double e = rel(y, ref_matmul(x, w.deq, M, K, N));
        CHECK(e < 1e-3, "q4 M=%d rel %.3g", M, e);
        CHECK(std::memcmp(y.data(), z.data(), y.size() * 4) == 0, "noalloc M=%d bits", M);
        for (int path_opt : {1, 2}) {
            OK(brik_set_option(ctx, BRIK_OPT_PATH, path_opt));
            OK(brik_matmul_t_q4(ctx, dx.as<float>(), w.nib.as<uint8_t>(), w.sc.as<uint16_t>(), w.mn.as<uint16_t>(),
                                dy.as<float>(), M, K, N));
        }
        OK(brik_set_option(ctx, BRIK_OPT_PATH, 0));
    }
    // q8 and q3 encoders and matmuls
    const size_t ne = (size_t)N * K;
    auto wf = uniform(ne);
    Dev src(ne * 4), codes(ne), s8(ne / 16), lo(ne / 4), hi(ne / 8), s3(ne / 16), m3(ne / 16), out(ne * 4);
    OK(brik_h2d(ctx, src.p, wf.data(), ne * 4));
    OK(brik_quantize_q8(ctx, src.as<float>(), codes.as<int8_t>(), s8.as<uint16_t>(), ne));
    OK(brik_quantize_q3(ctx, src.as<float>(), lo.as<uint32_t>(), hi.as<uint32_t>(), s3.as<uint16_t>(),
                        m3.as<uint16_t>(), ne));
    for (int M : {1, 5, 40}) {
        auto x = uniform((size_t)M * K);
        Dev dx((size_t)M * K * 4), dy((size_t)M * N * 4);
        OK(brik_h2d(ctx, dx.p, x.data(), x.size() * 4));
        OK(brik_dequant_q8_f32(ctx, codes.as<int8_t>(), s8.as<uint16_t>(), out.as<float>(), ne));
        OK(brik_matmul_t_q8(ctx, dx.as<float>(), codes.as<int8_t>(), s8.as<uint16_t>(), dy.as<float>(), M, K, N));
        OK(brik_sync(ctx));
        double e = rel(download<float>(dy.p, (size_t)M * N), ref_matmul(x, download<float>(out.p, ne), M, K, N));
        CHECK(e < 1e-3, "q8 M=%d rel %.3g", M, e);
        OK(brik_dequant_q3_f32(ctx, lo.as<uint32_t>(), hi.as<uint32_t>(), s3.as<uint16_t>(), m3.as<uint16_t>(),
                               out.as<float>(), ne));
        OK(brik_matmul_t_q3(ctx, dx.as<float>(), lo.as<uint32_t>(), hi.as<uint32_t>(), s3.as<uint16_t>(),
                            m3.as<uint16_t>(), dy.as<float>(), M, K, N));
        OK(brik_sync(ctx));
        e = rel(download<float>(dy.p, (size_t)M * N), ref_matmul(x, download<float>(out.p, ne), M, K, N));
        CHECK(e < 1e-3, "q3 M=%d rel %.3g", M, e);
    }
    // contract violations come back as error codes
    Dev dx(K * 4 + 16), dy(N * 4 + 16);
    CHECK(brik_matmul_t_q4(ctx, dx.as<float>(), w.nib.as<uint8_t>(), w.sc.as<uint16_t>(), w.mn.as<uint16_t>(),
                           dy.as<float>(), 1, 100, N) == BRIK_EINVAL, "K %% 32");
    CHECK(brik_matmul_t_q4(ctx, dx.at<float>(4), w.nib.as<uint8_t>(), w.sc.as<uint16_t>(), w.mn.as<uint16_t>(),
                           dy.as<float>(), 1, K, N) == BRIK_EALIGN, "misaligned x");
    CHECK(brik_matmul_t_q4(ctx, dx.as<float>(), nullptr, w.sc.as<uint16_t>(), w.mn.as<uint16_t>(),
                           dy.as<float>(), 1, K, N) == BRIK_EINVAL, "null plane");
    CHECK(brik_matmul_t_q4(ctx, dx.as<float>(), w.nib.as<uint8_t>(), w.sc.as<uint16_t>(), w.mn.as<uint16_t>(),
                           dy.as<float>(), -1, K, N) == BRIK_EINVAL, "negative M");
    for (int key = 1; key <= 7; ++key) OK(brik_set_option(ctx, key, 0));
    CHECK(brik_set_option(ctx, 999, 1) != BRIK_OK, "unknown option");
}

brik_gemv_job job(const Q4& w, const Dev& x, const Dev& y)
{
    return brik_gemv_job{x.as<float>(), w.nib.p, nullptr, w.sc.as<uint16_t>(), w.mn.as<uint16_t>(), y.as<float>(),
                         w.K, w.N};
}

void plans()
{
    const int K = 512;
    Q4 a(256, K), b(128, K), c(64, K);
    auto x = uniform(K);
    Dev dx(K * 4), ya(256 * 4), yb(128 * 4), yc(64 * 4), ref(256 * 4);
    OK(brik_h2d(ctx, dx.p, x.data(), K * 4));
    brik_gemv_job jobs[3] = {job(a, dx, ya), job(b, dx, yb), job(c, dx, yc)};
    brik_gemv_plan* p = nullptr;
    OK(brik_gemv_plan_create(ctx, BRIK_FMT_Q4, jobs, 3, &p));
    for (int i = 0; i < 3; ++i) OK(brik_gemv_plan_run(ctx, p));
    OK(brik_matmul_t_q4(ctx, dx.as<float>(), a.nib.as<uint8_t>(), a.sc.as<uint16_t>(), a.mn.as<uint16_t>(),
                        ref.as<float>(), 1, K, 256));
    OK(brik_sync(ctx));
    const double e = rel(download<float>(ya.p, 256), ref_matmul(x, a.deq, 1, K, 256));
    CHECK(e < 1e-5, "plan job 0 rel %.3g", e);
    brik_gemv_plan_destroy(ctx, p);
    CHECK(brik_gemv_plan_create(ctx, BRIK_FMT_Q4, jobs, 0, &p) == BRIK_EINVAL, "empty plan");
    CHECK(brik_gemv_plan_create(ctx, 5, jobs, 3, &p) == BRIK_EINVAL, "bad format");

    // fused jobs: RMSNorm input and a residual; SwiGLU input
    auto nw = uniform(K, 0.5f, 1.5f);
    Dev dn(K * 4), dg(K * 4);
    OK(brik_h2d(ctx, dn.p, nw.data(), K * 4));
    OK(brik_h2d(ctx, dg.p, x.data(), K * 4));
    brik_gemv_job_ex ex[2] = {};
    ex[0].job = job(a, dx, ya); ex[0].norm_w = dn.as<float>(); ex[0].eps = 1e-6f; ex[0].res = ref.as<float>();
    ex[1].job = job(b, dx, yb); ex[1].gate = dg.as<float>(); ex[1].flags = BRIK_JOB_ACT_GELU;
    OK(brik_gemv_plan_create_ex(ctx, BRIK_FMT_Q4, ex, 2, &p));
    OK(brik_gemv_plan_run(ctx, p));
    brik_gemv_plan_destroy(ctx, p);

    // the linked GLU pair: gate/up 256 x 512 on rmsnorm(x), down 64 x 256 on swiglu(gate, up) + residual
    Q4 gate(256, K), up(256, K), down(64, 256);
    Dev gy(256 * 4), uy(256 * 4), dy(64 * 4), res(64 * 4);
    auto r = uniform(64);
    OK(brik_h2d(ctx, res.p, r.data(), 64 * 4));
    brik_gemv_job_ex g = {}, u = {}, dj = {};
    g.job = job(gate, dx, gy); g.norm_w = dn.as<float>(); g.eps = 1e-6f;
    u.job = job(up, dx, uy); u.norm_w = dn.as<float>(); u.eps = 1e-6f;
    dj.job = job(down, uy, dy); dj.gate = gy.as<float>(); dj.res = res.as<float>();
    for (int order = 0; order < 2; ++order) {
        brik_gemv_plan *gu = nullptr, *dp = nullptr;
        OK(brik_gemv_plan_create_glu(ctx, BRIK_FMT_Q4, &g, &u, &dj, &gu, &dp));
        for (int i = 0; i < 2; ++i) {
            OK(brik_gemv_plan_run(ctx, gu));
            OK(brik_gemv_plan_run(ctx, dp));
        }
        OK(brik_sync(ctx));
        if (order) { brik_gemv_plan_destroy(ctx, gu); brik_gemv_plan_destroy(ctx, dp); }
        else { brik_gemv_plan_destroy(ctx, dp); brik_gemv_plan_destroy(ctx, gu); }
    }
    auto dv = download<float>(dy.p, 64);
    bool finite = true;
    for (float v : dv) finite &= std::isfinite(v);
    CHECK(finite, "GLU pair output finite");

    // a plan large enough to stage x once per run (a separate staging launch)
    Q4 big(24576, 64);
    auto xb = uniform(64);
    Dev bx(64 * 4), by(24576 * 4);
    OK(brik_h2d(ctx, bx.p, xb.data(), 64 * 4));
    brik_gemv_job bj = job(big, bx, by);
    OK(brik_gemv_plan_create(ctx, BRIK_FMT_Q4, &bj, 1, &p));
    OK(brik_gemv_plan_run(ctx, p));
    OK(brik_sync(ctx));
    const double eb = rel(download<float>(by.p, 24576), ref_matmul(xb, big.deq, 1, 64, 24576));
    CHECK(eb < 1e-5, "pre-staged plan rel %.3g", eb);
    brik_gemv_plan_destroy(ctx, p);

    // graph of a matmul and a plan, replayed
    OK(brik_gemv_plan_create(ctx, BRIK_FMT_Q4, jobs, 3, &p));
    OK(brik_gemv_plan_run(ctx, p));
    OK(brik_sync(ctx));
    brik_graph* gr = nullptr;
    OK(brik_graph_begin(ctx));
    OK(brik_matmul_t_q4(ctx, dx.as<float>(), a.nib.as<uint8_t>(), a.sc.as<uint16_t>(), a.mn.as<uint16_t>(),
                        ref.as<float>(), 1, K, 256));
    OK(brik_gemv_plan_run(ctx, p));
    void* during = nullptr;
    CHECK(brik_alloc(ctx, 64, &during) != BRIK_OK && during == nullptr, "allocation refused while capturing");
    OK(brik_graph_end(ctx, &gr));
    for (int i = 0; i < 3; ++i) OK(brik_graph_launch(ctx, gr));
    OK(brik_sync(ctx));
    brik_graph_destroy(ctx, gr);
    brik_gemv_plan_destroy(ctx, p);
}

void misc()
{
    // fences: an asynchronous readback
    Dev d(4096);
    std::vector<float> h(1024, 0.f), back(1024, 1.f);
    for (int i = 0; i < 1024; ++i) h[i] = (float)i;
    OK(brik_h2d(ctx, d.p, h.data(), 4096));
    brik_fence* f = nullptr;
    OK(brik_fence_record(ctx, &f));
    OK(brik_fence_d2h(f, back.data(), d.p, 4096));
    CHECK(back == h, "fence readback");
    CHECK(brik_fence_error(f) != nullptr, "fence error string");
    brik_fence_destroy(f);

    // top-k over logits with a penalty and softcap
    const int n = 5000, k = 8;
    auto lg = uniform(n, -5.f, 5.f);
    std::vector<int32_t> recent = {1, 7, 4999};
    Dev dl(n * 4), dr(recent.size() * 4), ids(k * 4), vals(k * 4);
    OK(brik_h2d(ctx, dl.p, lg.data(), n * 4));
    OK(brik_h2d(ctx, dr.p, recent.data(), recent.size() * 4));
    OK(brik_logits_topk(ctx, dl.as<float>(), n, dr.as<int32_t>(), 3, 1.3f, 30.f, k, ids.as<int32_t>(),
                        vals.as<float>()));
    OK(brik_sync(ctx));
    auto v = download<float>(vals.p, k);
    for (int i = 1; i < k; ++i) CHECK(v[i - 1] >= v[i], "top-k order");
    CHECK(brik_logits_topk(ctx, dl.as<float>(), n, nullptr, 0, 1.f, 0.f, 0, ids.as<int32_t>(), vals.as<float>()) ==
              BRIK_EINVAL, "k = 0");

    // LM head + top-k
    Q4 head(512, 256);
    auto x = uniform(256);
    Dev dx(256 * 4);
    OK(brik_h2d(ctx, dx.p, x.data(), 256 * 4));
    OK(brik_lm_head_topk_q4(ctx, dx.as<float>(), head.nib.as<uint8_t>(), head.sc.as<uint16_t>(),
                            head.mn.as<uint16_t>(), 256, 512, nullptr, 0, 1.f, 0.f, 4, ids.as<int32_t>(),
                            vals.as<float>()));

    // MoE: 4 experts, rows 10 / 0 / 15 / 15
    const int E = 4, N = 64, K = 512, R = 40;
    Q4 moe(E * N, K), moe2(E * N, K);
    std::vector<int32_t> off = {0, 10, 10, 25, 40};
    auto xm = uniform((size_t)R * K);
    Dev doff(off.size() * 4), dxm((size_t)R * K * 4), ya((size_t)R * N * 4), yb((size_t)R * N * 4);
    OK(brik_h2d(ctx, doff.p, off.data(), off.size() * 4));
    OK(brik_h2d(ctx, dxm.p, xm.data(), xm.size() * 4));
    OK(brik_moe_matmul_t_q4(ctx, dxm.as<float>(), doff.as<int32_t>(), moe.nib.as<uint8_t>(), moe.sc.as<uint16_t>(),
                            moe.mn.as<uint16_t>(), ya.as<float>(), E, R, K, N));
    OK(brik_moe_matmul_t_q4_x2(ctx, dxm.as<float>(), doff.as<int32_t>(), moe.nib.as<uint8_t>(), moe.sc.as<uint16_t>(),
                               moe.mn.as<uint16_t>(), yb.as<float>(), moe2.nib.as<uint8_t>(), moe2.sc.as<uint16_t>(),
                               moe2.mn.as<uint16_t>(), ya.as<float>(), E, R, K, N));
    OK(brik_sync(ctx));
    {
        // expert 2's rows [10, 25) against its weights
        auto y = download<float>(yb.p, (size_t)R * N);
        std::vector<float> xe(xm.begin() + 10 * K, xm.begin() + 25 * K);
        std::vector<float> we(moe.deq.begin() + (size_t)2 * N * K, moe.deq.begin() + (size_t)3 * N * K);
        std::vector<float> ye(y.begin() + 10 * N, y.begin() + 25 * N);
        const double e = rel(ye, ref_matmul(xe, we, 15, K, N));
        CHECK(e < 1e-3, "MoE expert 2 rel %.3g", e);
    }

    // convolution, f16 weights, f16 decode
    const int Cin = 32, H = 8, W = 8, Cout = 32;
    Q4 cw(Cout, Cin * 9);
    auto in = uniform((size_t)Cin * H * W), bias = uniform(Cout);
    Dev din(in.size() * 4), db(Cout * 4), dout((size_t)Cout * H * W * 4);
    OK(brik_h2d(ctx, din.p, in.data(), in.size() * 4));
    OK(brik_h2d(ctx, db.p, bias.data(), Cout * 4));
    OK(brik_conv2d_q4(ctx, din.as<float>(), cw.nib.as<uint8_t>(), cw.sc.as<uint16_t>(), cw.mn.as<uint16_t>(),
                      db.as<float>(), dout.as<float>(), Cin, H, W, Cout, 3, 3, 1, 1));
    std::vector<uint16_t> wh((size_t)128 * 256);
    for (auto& e : wh) e = (uint16_t)(0x3000 + (rng() & 0x7ff));    // f16 values in [0.125, 0.25)
    Dev dw(wh.size() * 2), wf(wh.size() * 4), xf(64 * 256 * 4), yf(64 * 128 * 4);
    auto xx = uniform(64 * 256);
    OK(brik_h2d(ctx, dw.p, wh.data(), wh.size() * 2));
    OK(brik_h2d(ctx, xf.p, xx.data(), xx.size() * 4));
    OK(brik_f16_to_f32(ctx, dw.as<uint16_t>(), wf.as<float>(), wh.size()));
    for (int M : {1, 64}) OK(brik_matmul_t_f16w(ctx, xf.as<float>(), dw.as<uint16_t>(), yf.as<float>(), M, 256, 128));
    OK(brik_sync(ctx));

    float ms = 0;
    OK(brik_timer_begin(ctx));
    OK(brik_timer_end(ctx, &ms));
    char stage[64] = {0};
    OK(brik_self_validate(ctx, stage, sizeof stage));
}

}  // namespace

int main(int argc, char** argv)
{
    host_checks();
    int ndev = 0;
    const bool nodev = argc > 1 && std::strcmp(argv[1], "nodev") == 0;
    if (nodev || brik_device_count(&ndev) != BRIK_OK || ndev == 0) {
        std::printf("host checks only (no device): %d failure(s)\n", fails);
        return fails ? 1 : 0;
    }
    for (int round = 0; round < 2; ++round) {
        OK(brik_create(0, &ctx));
        if (!ctx) return 1;
        std::printf("round %d: copies\n", round); std::fflush(stdout);
        copies();
        std::printf("round %d: matmuls\n", round); std::fflush(stdout);
        matmuls();
        std::printf("round %d: plans\n", round); std::fflush(stdout);
        plans();
        std::printf("round %d: misc\n", round); std::fflush(stdout);
        misc();
        OK(brik_sync(ctx));
        brik_destroy(ctx);
        ctx = nullptr;
    }
    // a context destroyed while a capture is still open, then a fresh one
    brik_ctx* c2 = nullptr;
    CHECK(brik_create(0, &c2) == BRIK_OK, "create for the open-capture case");
    if (c2) {
        CHECK(brik_graph_begin(c2) == BRIK_OK, "graph_begin");
        brik_destroy(c2);
    }
    CHECK(brik_create(0, &c2) == BRIK_OK, "create after destroying an open capture");
    if (c2) brik_destroy(c2);
    std::printf("device checks done: %d failure(s)\n", fails);
    return fails ? 1 : 0;
}
