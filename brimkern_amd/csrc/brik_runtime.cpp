// libbrik.so — C-ABI runtime over the gfx950 code object of the quantized matmul kernels.
//
// The code object (brik_gfx950.hsaco, built with `hipcc --genco --offload-arch=gfx950`) is
// embedded in this library by brik_embed.S and loaded with hipModuleLoadData; kernels are launched
// with hipModuleLaunchKernel on the context's own stream. Host API surface: device selection,
// hipMalloc/hipFree, hipMemcpy(Async), module load + launch, events for timing.
#include "../../include/brik.h"
#include "kernels/stage_abi.h"

#include <hip/hip_runtime_api.h>

#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <deque>
#include <new>
#include <vector>
#include <algorithm>
#include <cmath>

extern "C" const unsigned char brik_hsaco_begin[];
extern "C" const unsigned char brik_hsaco_end[];
// brik_scratch.hip: device address of the fixed scratch array on the current device (a hipError_t)
extern "C" int brik_scratch_resolve(int device, void** out, size_t* bytes);

namespace {

enum Kern {
    K_DEQ_Q8, K_DEQ_Q4, K_DEQ_Q3,
    K_XPREP,
    K_TOPK_PREP, K_TOPK_SELECT,
    K_FILL_ZERO,
    K_QUANT_Q8, K_QUANT_Q4, K_QUANT_Q3, K_F16_TO_F32,
    K_CONV_Q8, K_CONV_Q4, K_XPREP_IM2COL, K_CONV_OUT, K_CONV_CHANMAX, K_XPREP_IM2COL3,
    K_GEMV_F16W_V8, K_GEMV_F16W_V4, K_GEMM_F16W,
    K_GEMV_STAGE_Q8, K_GEMV_STAGE_Q4, K_GEMV_STAGE_Q3, K_GEMV_STAGE1_Q4, K_GEMV_STAGE1_Q3,
    K_SPLITK_REDUCE,
    K_COUNT
};

const char* const kKernelNames[K_COUNT] = {
    "brik_dequant_q8", "brik_dequant_q4", "brik_dequant_q3",
    "brik_xprep_f16",
    "brik_topk_prep", "brik_topk_select",
    "brik_fill_zero",
    "brik_encode_q8", "brik_encode_q4", "brik_encode_q3", "brik_f16_decode",
    "brik_conv2d_direct_q8", "brik_conv2d_direct_q4", "brik_xprep_im2col_f16", "brik_conv_out",
    "brik_conv_chanmax", "brik_xprep_im2col3_f16",
    "brik_gemv_f16w_v8", "brik_gemv_f16w_v4", "brik_gemm_f16w",
    "brik_gemv_stage_q8", "brik_gemv_stage_q4", "brik_gemv_stage_q3", "brik_gemv_stage1_q4", "brik_gemv_stage1_q3",
    "brik_splitk_reduce",
};

// GEMV variants {team, r, u, d}, in the order of BRIK_GEMV_FMT in gemv.hip: TEAM lanes per row team,
// R rows per team, U groups per pipeline step, pipeline depth D; kernels brik_gemv_<fmt>_t<T>_r<R>_u<U>_d<D>
// (one matrix) and brik_gemvg_<fmt>_... (grouped job table).
struct GemvVariant {
    int team, r, u, d;
    constexpr int rpi() const { return (256 / team) * r; }      // rows per block iteration
    // LDS of a block past the staged x: TEAM partial sums for each of `rows` rows
    constexpr size_t extra_lds(long rows) const { return sizeof(float) * (size_t)rows * team; }
};
constexpr GemvVariant kGemvVariants[] = {{16, 2, 1, 2}, {16, 2, 1, 3}, {16, 2, 1, 4}, {16, 4, 1, 2},
                                         {16, 2, 2, 2}, {32, 2, 1, 3}, {64, 1, 1, 3}, {16, 2, 5, 2},
                                         {16, 1, 5, 2}, {16, 1, 2, 2}, {32, 1, 1, 2}};
constexpr int kNumGemvVariants = sizeof(kGemvVariants) / sizeof(kGemvVariants[0]);
const char* const kFmtNames[3] = {"q8", "q4", "q3"};
// GLU pair kernels brik_gemvp_<fmt>_t16_r2_u1_d2_n512 (q4, q3): 512-thread blocks of 32 teams of 16
// lanes, each team with one row of gate and the same row of up, so a block covers 32 rows of each (one
// quantization group of down's input) with as many waves as two blocks of the unpaired gate/up plan.
constexpr GemvVariant kGluVariant = {16, 2, 1, 2};
constexpr int kGluThreads = 512;
constexpr int kGluRows = 32;   // rows of each matrix per block
static_assert(kGluThreads / kGluVariant.team * kGluVariant.r == 2 * kGluRows, "GLU block rows");
// the pair launch's blocks past the whole groups: 8 teams of 64 lanes, one row of each matrix per team
constexpr int kGluTailRows = 8;
static_assert(kGluThreads / 64 * kGluVariant.r == 2 * kGluTailRows, "GLU tail block rows");

// the variant of the LM-head kernels brik_gemvh_<fmt>_t16_r2_u5_d2 (the one a staged single q4 / q3
// matrix runs)
constexpr int kHeadVariant = 7;

constexpr int kGroup = 32;
// GEMM block tiles (BM rows x 32 TN NW columns, NW waves), in the order of BRIK_GEMM_FMT in gemm.hip:
// brik_gemm_<fmt>_<BM>x<TN> (NW = 4) and brik_gemm_<fmt>_<BM>x<TN>w8 (NW = 8).
// pf: steps of W prefetched ahead (kernel suffix p<pf> when above 1)
struct GemmTile {
    int bm, tn, nw, pf;
    int bn() const { return 32 * tn * nw; }
    unsigned threads() const { return 64u * (unsigned)nw; }
};
constexpr GemmTile kGemmTiles[] = {{128, 2, 4, 1}, {128, 1, 4, 1}, {128, 3, 4, 1}, {64, 2, 4, 1}, {64, 1, 4, 1},
                                   {64, 3, 4, 1},  {32, 2, 4, 1},  {32, 1, 4, 1},  {32, 3, 4, 1}, {96, 2, 4, 1},
                                   {96, 1, 4, 1},  {96, 3, 4, 1},  {128, 1, 8, 1}, {96, 1, 8, 1}, {64, 1, 8, 1},
                                   {32, 1, 8, 1},  {64, 2, 8, 1},  {32, 1, 8, 4},  {64, 1, 8, 3}, {32, 1, 4, 4},
                                   {64, 1, 4, 3},  {32, 1, 8, 2},  {64, 1, 8, 2}};
constexpr int kNumGemmTiles = sizeof(kGemmTiles) / sizeof(kGemmTiles[0]);

constexpr unsigned kCUs = 256;                 // MI355X compute units
constexpr long kGemmKPad = 256;                // staged activation rows are padded to this many halves
constexpr size_t kGemvMaxLds = 64 * 1024;      // dynamic LDS budget of one GEMV block
constexpr unsigned kGemvMaxBlocks = 16384;     // GEMV grid cap; blocks then loop over row sets
// target (rows x groups) per grouped-plan block and its row sets, at most: each block stages x once,
// so fewer, larger blocks spend less on staging (36-layer q4 set: 311 us at 32768 x 8 sets, 313.5 us
// at 16384 x 4, 321 us at 8192 x 4, 342 us at 4096 x 4)
constexpr double kPlanGroupRows = 32768;
constexpr long kPlanMaxSets = 8;
constexpr size_t kPlanPartialLds = 16384;      // LDS reserved for a plan block's lane partials
// Plans of at least this many rows stage every distinct input row once per run (a staging launch
// before the GEMV) and their blocks copy the staged image; with staging off the block critical path,
// smaller blocks stream better: the 36-layer q4 set measured 294 us at 8192 x 4 against 304 us at
// 32768 x 8 with per-block staging (a probe with the staging removed).
constexpr long kPrestageRows = 96L * 256;
constexpr unsigned kStageThreads = 1024;       // threads of a staging block (launch bounds of brik_gemv_stage_*)
constexpr double kPrestageGroupRows = 8192;
constexpr long kPrestageMaxSets = 4;
constexpr long kPrestageMinSets = 2;
// The last jobs of a pre-staged plan of many blocks run in single-set blocks, about this many of them
// (whole jobs): the launch's drain, where fewer blocks than the CUs hold remain, then ends on short
// blocks (36-layer q4 set, 3 rounds of alternating processes: 298.6-298.9 us per step with none,
// 297.9-298.2 with 256 or 768, 298.2-298.3 with 1536; two-set tail blocks were slower, 299.2-300.3 us).
constexpr long kPrestageTailBlocks = 512;
constexpr long kPlanMinBlocks = 1024;          // grouped-plan blocks, at least (while sets > 1)

enum Fmt { F_Q8 = 8, F_Q4 = 4, F_Q3 = 3 };

// LDS bytes of a staged activation row (xprep.h), per group plus one zero group: q8 / q3 96 limb
// bytes, an f32 sum and an int32 exponent; q4 96 bytes of digit planes and 16 bytes of sums and
// exponent. Then a flag, the RMSNorm factor and 16 reduction slots, 80 bytes (BRIK_XSTAGE_TAIL).
size_t gemv_lds(int K, Fmt f) { return (size_t)(f == F_Q8 ? 104 : 112) * (K / kGroup + 1) + 80; }
int fmt_index(int f) { return f == F_Q8 ? 0 : f == F_Q4 ? 1 : 2; }

}  // namespace

static_assert(sizeof(brik_gemv_block) == 128, "block table entry");

// A device buffer shared by the two plans of a GLU pair (the staged image of act(gate) * up), freed
// with the last of them.
struct SharedBuf {
    void* ptr = nullptr;
    int refs = 0;
};

struct brik_gemv_plan {
    hipFunction_t kernel;
    // grouped: [block table (brik_gemv_block per launch block) | stage inputs]; GLU pair: [gate job | up job]
    void* dev = nullptr;
    int njobs = 0;
    unsigned blocks = 0;
    size_t lds = 0;
    // staging pass of a large plan: `ninputs` distinct input rows, staged into `stage`
    hipFunction_t stager = nullptr;
    void* stage = nullptr;        // owned, unless `image` holds it
    int ninputs = 0;
    size_t inputs_off = 0;        // byte offset of the stage-input table in dev
    // GLU pairs: the producer (glu = true) writes the image in `image`, the consumer copies it as its
    // staged input (stage = image->ptr, no stager)
    bool glu = false;
    int act_flags = 0;
    int glu_full = 0;             // producer blocks that write whole groups of the image
    SharedBuf* image = nullptr;
};

struct brik_fence {
    int device = -1;
    hipEvent_t ev = nullptr;
    char err[256] = {0};
};

struct brik_graph {
    hipGraph_t graph = nullptr;
    hipGraphExec_t exec = nullptr;
    // the context's workspace generation when the capture ended: the recorded launches hold the
    // workspace addresses of that moment. Checked at launch only if the capture used a context
    // workspace (uses_ws): a graph of plans and no-allocation calls holds none of those addresses.
    unsigned long long ws_generation = 0;
    bool uses_ws = false;
};

struct brik_ctx {
    int device = -1;
    hipModule_t module = nullptr;
    hipFunction_t fn[K_COUNT] = {};
    hipFunction_t gemv[3][kNumGemvVariants] = {};
    hipFunction_t gemvg[3][kNumGemvVariants] = {};
    hipFunction_t gemvp[3] = {};                 // GLU pair kernels (q4, q3; q8 has none)
    hipFunction_t gemvh[3] = {};                 // LM heads with the top-k pre-work (q4, q3; variant kHeadVariant)
    hipFunction_t gemm[3][kNumGemmTiles] = {};
    hipFunction_t gemmg[kNumGemmTiles] = {};    // expert-grouped q4 kernels (brik_gemmg_q4_*)
    hipFunction_t gemmg_adapt[2] = {};           // brik_gemmg_q4_64a (4 waves), brik_gemmg_q4_64aw8 (8 waves)
    hipFunction_t gemm_f16[kNumGemmTiles] = {};   // f16-weight tiles (TN = 1, PF = 1 only; others null)
    hipFunction_t gemm_sk[3][3] = {};      // split-K few-row kernels, KSL = 2, 4, 8
    hipStream_t stream = nullptr;
    hipEvent_t ev_begin = nullptr, ev_end = nullptr;
    int opt_path = 0;
    int opt_variant = 0;   // 0 auto, else 1 + index into kGemvVariants
    int opt_tile = 0;      // 0 auto, else 1 + index into kGemmTiles
    int opt_plan_stage = 0;  // plans: 0 auto, 1 in-block staging, 2 staging launch
    int opt_plan_sets = 0;   // plans: 0 auto, else row sets per block
    int opt_splitk = 0;      // few-row GEMMs: 0 auto, 1 never split-K, 2 split-K whenever it applies
    int opt_gemv_blocks = 0; // single-matrix GEMV: 0 auto, else grid cap
    void* ws = nullptr;    // GEMM workspace: f16 activation rows, then per-row scales (grow-only)
    size_t ws_bytes = 0;
    void* tws = nullptr;   // top-k workspace: lane maxima, then LM-head logits (grow-only)
    size_t tws_bytes = 0;
    void* sws = nullptr;   // staged activation row of a large single-matrix GEMV (grow-only)
    size_t sws_bytes = 0;
    void* cws = nullptr;   // convolution workspace: the [pixels, Cout] GEMM output (grow-only)
    size_t cws_bytes = 0;
    void* pws = nullptr;   // split-K partial tiles [slice][row][column] f32 (grow-only)
    size_t pws_bytes = 0;

    // pinned staging ring of brik_h2d_async (allocated on first use): uploads in flight as
    // {offset, bytes, event} in issue order; events are recycled through a free list
    struct Upload {
        size_t off, len;
        hipEvent_t ev;
    };
    void* ring = nullptr;
    size_t ring_head = 0;
    std::deque<Upload> ring_inflight;
    std::vector<hipEvent_t> ring_events;

    // the device's fixed scratch array (brik_scratch.hip), resolved at creation; scratch_err holds the
    // hipError_t of a failed resolution, which only the no-allocation entry point reports
    void* scratch = nullptr;
    size_t scratch_bytes = 0;
    int scratch_err = 0;
    int last_path = 0;            // BRIK_PATH_* of the last matmul call (brik_last_path)
    bool graph_capturing = false;
    bool graph_used_ws = false;   // the open capture recorded a launch on a context workspace
    // bumped whenever a context workspace is freed and reallocated (ensure_buf): a graph recorded
    // before that replays addresses that are no longer the context's, so brik_graph_launch refuses it
    unsigned long long ws_generation = 0;
    char err[512] = {0};
};

namespace {

int fail(brik_ctx* c, int code, const char* fmt, ...)
{
    if (c) {
        va_list ap;
        va_start(ap, fmt);
        vsnprintf(c->err, sizeof c->err, fmt, ap);
        va_end(ap);
    }
    return code;
}

#define HIP_TRY(ctx, call)                                                                    \
    do {                                                                                      \
        hipError_t e_ = (call);                                                               \
        if (e_ != hipSuccess)                                                                 \
            return fail((ctx), e_ == hipErrorOutOfMemory ? BRIK_ENOMEM : BRIK_EHIP, "%s: %s", \
                        #call, hipGetErrorString(e_));                                        \
    } while (0)

#define HIP_TRY_RC(call)          \
    do {                          \
        const int r_ = (call);    \
        if (r_ != BRIK_OK) return r_; \
    } while (0)

bool aligned(const void* p, size_t a) { return (reinterpret_cast<uintptr_t>(p) & (a - 1)) == 0; }

int launch_fn(brik_ctx* c, hipFunction_t f, unsigned gx, unsigned gy, unsigned bx, size_t lds, void** args)
{
    if (gx == 0 || gy == 0) return BRIK_OK;
    HIP_TRY(c, hipSetDevice(c->device));
    HIP_TRY(c, hipModuleLaunchKernel(f, gx, gy, 1, bx, 1, 1, (unsigned)lds, c->stream, args, nullptr));
    return BRIK_OK;
}

int launch(brik_ctx* c, Kern k, unsigned gx, unsigned gy, unsigned bx, size_t lds, void** args)
{
    return launch_fn(c, c->fn[k], gx, gy, bx, lds, args);
}

// Shape + pointer validation shared by the three matmuls.
int check_mm(brik_ctx* c, const char* who, const float* x, const void* p0, const void* p1,
             const void* sc, const void* mn, const float* y, int M, int K, int N, Fmt f)
{
    if (!c) return BRIK_EINVAL;
    if (M < 0 || K < 0 || N < 0) return fail(c, BRIK_EINVAL, "%s: negative shape M=%d K=%d N=%d", who, M, K, N);
    if (K % kGroup) return fail(c, BRIK_EINVAL, "%s: K=%d is not a multiple of 32", who, K);
    if (M == 0 || N == 0) return BRIK_OK;
    if (!y) return fail(c, BRIK_EINVAL, "%s: y is null", who);
    if (!aligned(y, 4)) return fail(c, BRIK_EALIGN, "%s: y must be 4-byte aligned", who);
    if (K == 0) return BRIK_OK;
    if (!x || !p0 || !sc || (f != F_Q8 && !mn) || (f == F_Q3 && !p1))
        return fail(c, BRIK_EINVAL, "%s: null operand pointer", who);
    if (!aligned(x, 16)) return fail(c, BRIK_EALIGN, "%s: x must be 16-byte aligned", who);
    if (!aligned(p0, 16)) return fail(c, BRIK_EALIGN, "%s: code plane must be 16-byte aligned", who);
    if (f == F_Q3 && !aligned(p1, 8)) return fail(c, BRIK_EALIGN, "%s: q3 hi plane must be 8-byte aligned", who);
    if (!aligned(sc, 2) || (mn && !aligned(mn, 2)))
        return fail(c, BRIK_EALIGN, "%s: scales/mins must be 2-byte aligned", who);
    // each plane is addressed through one buffer resource (32-bit byte offsets); the largest
    // plane is the q8 code plane, N*K bytes
    if ((unsigned long long)N * (unsigned long long)K >= (1ull << 32))
        return fail(c, BRIK_EINVAL, "%s: N*K = %lld elements exceeds the 2^32 per-tensor limit", who, (long long)N * K);
    return BRIK_OK;
}

unsigned gemm_tiles(long n, int t) { return (unsigned)((n + t - 1) / t); }

// GEMM block tile (index into kGemmTiles).
// Dense (E == 0): the tile with the smallest modelled makespan, rounds x tile area x a small-tile
// penalty, where rounds = ceil(blocks / CUs) (every block of a round runs on its own compute unit).
// A 256-column tile runs as its 8-wave form (two waves per SIMD): measured on the M = 512, K = 2560, N = 9728 prefill shape
// (M = 512, K = 2560, N = 9728) with cold weights 44.9 us against 47.5 us for 96 x 256 with 4 waves,
// and 5-10 % faster at every other row count.
// Expert-grouped (MoE): 64-row tiles; 64 x 128 with 4 waves for K >= 2048 (16 or more K steps), else
// 64 x 256 with 8 waves. Measured on a 64-expert MoE layer (22-47 rows each), every tile forced, per
// call with the x staging: gate + up in one launch (K = 2048, N = 768) 53.7-55.7 us with the 4-wave
// tile against 60-65 us with the 8-wave one and 60-96 us for the others; down (K = 768, N = 2048)
// 29.4-30.6 us with the 8-wave tile against 32.8-33.1 with the 4-wave one and 33-61 us for the others;
// a single gate (K = 2048, N = 768) the same with either (32.3 / 32.7 us kernel time).
int gemm_tile(brik_ctx* c, long M, long N, long K, int E)
{
    if (c->opt_tile > 0) return c->opt_tile - 1;
    auto find = [](int bm, int tn, int nw, int pf = 1) {
        for (int t = 0; t < kNumGemmTiles; ++t)
            if (kGemmTiles[t].bm == bm && kGemmTiles[t].tn == tn && kGemmTiles[t].nw == nw && kGemmTiles[t].pf == pf)
                return t;
        return 0;
    };
    if (E > 0) return K >= 2048 ? find(64, 1, 4) : find(64, 1, 8);
    // the modelled makespan over the 4-wave tiles, or (only256) over the 256-column ones
    auto pick = [&](bool only256, double& blocks_of_best) {
        int best = 0;
        double best_cost = 0;
        for (int t = 0; t < kNumGemmTiles; ++t) {
            GemmTile g = kGemmTiles[t];
            if (g.nw != 4 || g.pf != 1 || (only256 && (g.tn != 2 || g.bm < 64))) continue;
            const double blocks = (double)gemm_tiles(M, g.bm) * gemm_tiles(N, g.bn());
            const double rounds = std::ceil(blocks / kCUs);
            const double penalty = g.bm == 128 ? 1.0 : g.bm == 96 ? 1.1 : g.bm == 64 ? 1.3 : 1.8;
            const double cost = rounds * g.bm * (double)g.bn() * penalty;
            if (best_cost == 0 || cost < best_cost) {
                best = t;
                best_cost = cost;
                blocks_of_best = blocks;
            }
        }
        return best;
    };
    // Launches of at least one round of 64- to 128-row 256-column tiles keep to those (8-wave forms): on
    // K = 2560, N = 9728 at M = 1024 and 2048 the all-tile model picked a 128 x 128 tile that ran 90 and
    // 155-167 us against 80-81 us (96 x 256) and 139.5 us (128 x 256).
    double blocks = 0;
    int best = pick(true, blocks);
    if (blocks < kCUs) best = pick(false, blocks);
    // One round of 128 x 256 tiles that fills most of the CUs beats more blocks of fewer rows: a
    // 128-row block runs its tile at about 1.37x the per-CU rate of a 96-row one (x fragments and
    // dequantized codes each feed more MFMAs). Measured at K = 2560, N = 9728 (graph-free calls, 8 weight
    // copies): M = 512 42.7-43.0 us against 44.1-44.3 (96 x 256); M = 640 47.3 against 55-59 (model's
    // pick) and 72.5 (96 x 256); M = 768 52.5 against 52.5-54 and 74; at 76-114 blocks (M = 256, 384)
    // the smaller tiles stay ahead (28-35 us against 37-40).
    const double b128 = (double)gemm_tiles(M, 128) * gemm_tiles(N, 256);
    if (b128 >= 0.55 * kCUs && b128 <= kCUs) return find(128, 1, 8);
    const GemmTile& g = kGemmTiles[best];
    return g.tn == 2 ? find(g.bm, 1, 8) : best;     // the 8-wave form of a 256-column tile
}

// Grow a context workspace to at least `bytes`. Earlier launches on the context stream may still
// read the old buffer, so the stream is drained before it is freed.
int ensure_buf(brik_ctx* c, void*& buf, size_t& have, size_t bytes)
{
    if (c->graph_capturing) c->graph_used_ws = true;
    if (have >= bytes) return BRIK_OK;
    if (c->graph_capturing)
        return fail(c, BRIK_EINVAL, "a workspace would grow during graph capture: run the same calls once "
                                    "before brik_graph_begin");
    if (buf) {
        HIP_TRY(c, hipStreamSynchronize(c->stream));
        HIP_TRY(c, hipFree(buf));
        buf = nullptr;
        have = 0;
        ++c->ws_generation;
    }
    bytes = (bytes + (1u << 20) - 1) & ~(size_t)((1u << 20) - 1);
    HIP_TRY(c, hipMalloc(&buf, bytes));
    have = bytes;
    return BRIK_OK;
}

// Device memory a call uses beyond its inputs and outputs. By default the context workspaces above
// (grown with hipMalloc on demand); the no-allocation entry point passes a fixed buffer instead, and
// a call that would need more than it holds fails before anything is enqueued.
struct Scratch {
    void* p = nullptr;
    size_t bytes = 0;
};

int take_scratch(brik_ctx* c, const Scratch* fixed, void*& buf, size_t& have, size_t bytes, void*& out)
{
    if (!fixed) {
        HIP_TRY_RC(ensure_buf(c, buf, have, bytes));
        out = buf;
        return BRIK_OK;
    }
    if (bytes > fixed->bytes)
        return fail(c, BRIK_EINVAL, "no-allocation call: needs %zu bytes of scratch, the fixed buffer holds %zu",
                    bytes, fixed->bytes);
    out = fixed->p;
    return BRIK_OK;
}

// y[0, n) = 0 on the context stream (a kernel, so graph capture records no memset node).
int fill_zero(brik_ctx* c, float* y, size_t n)
{
    if (n == 0) return BRIK_OK;
    size_t blocks = (n + 255) / 256;
    blocks = blocks < 4096 ? blocks : 4096;
    void* args[] = {&y, &n};
    return launch(c, K_FILL_ZERO, (unsigned)blocks, 1, 256, 0, args);
}

// Bytes of `rows` staged f16 activation rows of K (padded to Kp halves) and their row scales.
size_t gemm_stage_bytes(long rows, long K, long& Kp)
{
    Kp = (K + kGemmKPad - 1) / kGemmKPad * kGemmKPad;
    return (size_t)rows * Kp * 2 + 4 * (size_t)rows;
}

// Workspace for `rows` staged f16 activation rows of K (padded to Kp) and their row scales.
int gemm_stage_ws(brik_ctx* c, int rows, int K, long& Kp, uint16_t*& xh, float*& rscale,
                  const Scratch* fixed = nullptr)
{
    const size_t bytes = gemm_stage_bytes(rows, K, Kp);
    const size_t xbytes = (size_t)rows * Kp * 2;
    if (xbytes >= (1ull << 31))
        return fail(c, BRIK_EINVAL, "matmul: %d rows x K=%d exceed the 2 GiB staged-activation limit", rows, K);
    void* p = nullptr;
    HIP_TRY_RC(take_scratch(c, fixed, c->ws, c->ws_bytes, bytes, p));
    xh = static_cast<uint16_t*>(p);
    rscale = reinterpret_cast<float*>(static_cast<char*>(p) + xbytes);
    return BRIK_OK;
}

// Grid of brik_xprep_f16 (gemm.hip): one 256-thread block per row, or per four rows when a staged
// row holds at most 2048 halves (one wave per row); at most 65536 blocks, which loop over the rest.
unsigned xprep_grid(long rows, long Kp)
{
    const long blocks = Kp <= 2048 ? (rows + 3) / 4 : rows;
    return (unsigned)(blocks < 65536 ? blocks : 65536);
}

// M >= 2 (dense): the cheapest of three paths by a cost model fitted per format on the Qwen3-4B shapes
// (k/v, gate, down for q8 and q3; all six for q4) at M = 2, 4, 8, 15, each path timed as graph-replayed
// back-to-back calls (us per call, launches included; W bytes = the packed planes):
// GEMV (grid.y = M: every activation row streams W again, rows after the first mostly from the 256 MB
// last-level cache): 3.5 + M (0.35 min(1, N / 1024) + W bytes / (7.8 TB/s q4, 6.0 q8 / q3)); the
// per-row latency term is that of rows whose blocks fill the chip (N >= 1024), smaller rows overlap.
// Tiled GEMM: 5 + max(c per 128-deep K step, which is what its few-row tiles spend in issue latency on
// one wave per SIMD (c = 0.70 us q4, 0.83 q8, 0.86 q3), 2MNK at 1 PFLOP/s).
// Split-K (few rows, below): 7.7 us of launches (x staging, the kernel, the slice sum), 0.15 us per K step,
// W at 3.4 TB/s (q4), 4.8 (q8), 2.4 (q3; its unpacking), 0.15 us per row.
// Over the 66 measured points the choice costs 0.9 us in total against the fastest path (the q4-only fit
// it replaces, which took the tiled GEMM for q8 / q3 gate shapes at M = 4-15: 38.8 us). M = 32,
// K = 9728, N = 2560: split-K 30 us against 94 tiled (eager timing). The tiled GEMM keeps M > 64.
enum SmallMPath { SM_GEMV, SM_SPLITK, SM_TILED };
constexpr long kSplitKMaxRows = 64;

SmallMPath small_m_path(Fmt f, long M, long K, long N)
{
    const double nk = (double)N * K;
    const double wbytes = f == F_Q4 ? nk * (0.5 + 4.0 / kGroup) : f == F_Q8 ? nk * (1.0 + 2.0 / kGroup)
                                                                            : nk * (0.375 + 4.0 / kGroup);
    const double steps = (double)((K + 2 * 128 - 1) / (2 * 128) * 2);
    const double gemv_bw = f == F_Q4 ? 7.8e6 : 6.0e6;                   // bytes per us
    const double tiled_step = f == F_Q4 ? 0.70 : f == F_Q8 ? 0.83 : 0.86;
    const double sk_bw = f == F_Q4 ? 3.4e6 : f == F_Q8 ? 4.8e6 : 2.4e6;
    const double gemv_us = 3.5 + (double)M * (0.35 * std::min(1.0, N / 1024.0) + wbytes / gemv_bw);
    const double tiled_us = 5.0 + std::max(tiled_step * steps, 2.0 * M * nk / 1e9);
    const double sk_us = M <= kSplitKMaxRows ? 7.7 + 0.15 * steps + wbytes / sk_bw + 0.15 * M : 1e30;
    if (gemv_us <= sk_us && gemv_us <= tiled_us) return SM_GEMV;
    return sk_us <= tiled_us ? SM_SPLITK : SM_TILED;
}

bool gemv_cheaper(Fmt f, long M, long K, long N) { return small_m_path(f, M, K, N) == SM_GEMV; }

// Split-K few-row kernel (brik_gemm_sk_<fmt>_k<KSL>): 32 x 128 tiles, each over K slices of at most
// KSL steps of 128. The slices are sized so the launch has about 1024 blocks (four per CU): the largest
// KSL of {8, 4, 2} that still gives that many, then as many slices as the K steps need.
constexpr int kSkTarget = 1024;
struct SplitK {
    int k;               // index of KSL in {2, 4, 8}
    unsigned gx, gy, gz;
};

SplitK splitk_shape(long rows, int K, int N, int E)
{
    const long steps = (K + 255) / 256 * 2;
    SplitK p;
    p.gx = (unsigned)((N + 127) / 128);
    p.gy = (unsigned)((rows + 31) / 32 + E);
    const long tiles = (long)p.gx * p.gy;
    const long want = (kSkTarget + tiles - 1) / tiles;           // slices wanted
    p.k = 0;
    for (int k = 2; k >= 0; --k)
        if ((steps + (2 << k) - 1) / (2 << k) >= want || k == 0) { p.k = k; break; }
    p.gz = (unsigned)((steps + (2 << p.k) - 1) / (2 << p.k));
    return p;
}

// Whether a GEMM takes the split-K kernel: dense launches of few rows where the cost model above prefers
// it, unless a tile is forced or the option says so. Expert-grouped launches keep the tiled kernel: on
// the 64-expert layer (20-50 rows per expert) split-K measured slower (gate 62 us against 42, down 50
// against 35: experts past 32 rows read their weights twice, and the two-slice gate adds the slice sum).
bool use_splitk(const brik_ctx* c, Fmt f, long rows, int K, int N, int E)
{
    if (c->opt_tile > 0 || c->opt_splitk == 1) return false;
    if (c->opt_splitk == 2) return true;
    return E == 0 && rows <= kSplitKMaxRows && small_m_path(f, rows, K, N) == SM_SPLITK;
}

// Bytes of the split-K partial tiles a GEMM over `rows` rows writes (0: no split-K, or one slice).
size_t splitk_part_bytes(const brik_ctx* c, Fmt f, long rows, int K, int N, int E)
{
    if (!use_splitk(c, f, rows, K, N, E)) return 0;
    const SplitK p = splitk_shape(rows, K, N, E);
    return p.gz > 1 ? (size_t)p.gz * rows * N * 4 : 0;
}

// Offset of the split-K partial tiles in a fixed scratch: after the staged rows, 256-byte aligned.
size_t splitk_part_off(long rows, int K)
{
    long Kp;
    return (gemm_stage_bytes(rows, K, Kp) + 255) & ~(size_t)255;
}

int gemm_splitk(brik_ctx* c, Fmt f, const uint16_t* xh, const float* rscale, const void* p0, const void* p1,
                const void* sc, const void* mn, float* y, int rows, int K, int N, const int* row_off, int E,
                const Scratch* fixed)
{
    const SplitK p = splitk_shape(rows, K, N, E);
    float* part = nullptr;
    if (p.gz > 1) {
        const size_t bytes = (size_t)p.gz * rows * N * 4;
        if (fixed) {
            // the no-allocation entry point: after the staged rows in the same fixed buffer (gemm checked
            // that both fit before enqueueing anything)
            const size_t off = splitk_part_off(rows, K);
            if (off + bytes > fixed->bytes)
                return fail(c, BRIK_EINVAL, "no-allocation call: needs %zu bytes of scratch, the fixed buffer "
                            "holds %zu", off + bytes, fixed->bytes);
            part = reinterpret_cast<float*>(static_cast<char*>(fixed->p) + off);
        } else {
            void* pw = nullptr;
            HIP_TRY_RC(take_scratch(c, nullptr, c->pws, c->pws_bytes, bytes, pw));
            part = static_cast<float*>(pw);
        }
    }
    int Mi = rows, Ki = K, Ni = N, Ei = E;
    void* args[] = {&xh, &rscale, &p0, &p1, &sc, &mn, &y, &Mi, &Ki, &Ni, &row_off, &Ei, &part};
    hipFunction_t fn = c->gemm_sk[fmt_index(f)][p.k];
    HIP_TRY(c, hipSetDevice(c->device));
    HIP_TRY(c, hipModuleLaunchKernel(fn, p.gx, p.gy, p.gz, 256, 1, 1, 0, c->stream, args, nullptr));
    if (p.gz == 1) return BRIK_OK;
    // the slices' partial tiles, summed in slice order
    size_t n = (size_t)rows * N;
    int ks = (int)p.gz;
    const size_t blocks = ((n + 3) / 4 + 255) / 256;
    void* rargs[] = {&part, &y, &n, &ks};
    return launch(c, K_SPLITK_REDUCE, (unsigned)(blocks < 2048 ? blocks : 2048), 1, 256, 0, rargs);
}

// A second q4 weight tensor multiplied by the same staged rows in the same launch (an MoE layer's gate
// and up projections): its codes, scales, mins and output.
struct WeightPair {
    const void* p0;
    const void* sc;
    const void* mn;
    float* y;
};

// The tile kernel over staged rows: dense when row_off is null, expert-grouped (q4) otherwise; `pair`
// (grouped only) adds the second tensor as blockIdx.z == 1.
// trans (dense, not split-K): y is [N, rows], y[n, m] = (x . W^T)[m, n] + tbias[n] (tbias may be null).
int gemm_run(brik_ctx* c, Fmt f, const uint16_t* xh, const float* rscale, const void* p0, const void* p1,
             const void* sc, const void* mn, float* y, int rows, int K, int N, const int* row_off, int E,
             const Scratch* fixed = nullptr, const WeightPair* pair = nullptr, const float* tbias = nullptr,
             int trans = 0)
{
    if (use_splitk(c, f, rows, K, N, E)) {
        c->last_path = BRIK_PATH_SPLITK;
        HIP_TRY_RC(gemm_splitk(c, f, xh, rscale, p0, p1, sc, mn, y, rows, K, N, row_off, E, fixed));
        if (!pair) return BRIK_OK;
        return gemm_splitk(c, f, xh, rscale, pair->p0, p1, pair->sc, pair->mn, pair->y, rows, K, N, row_off, E,
                           fixed);
    }
    c->last_path = BRIK_PATH_TILED;
    int Mi = rows, Ki = K, Ni = N, Ei = E;
    const int t = gemm_tile(c, rows, N, K, E);
    const GemmTile& gt = kGemmTiles[t];
    const int bn = gt.bn();
    if (!row_off) {
        void* args[] = {&xh, &rscale, &p0, &p1, &sc, &mn, &y, &Mi, &Ki, &Ni, &row_off, &Ei, &tbias, &trans};
        return launch_fn(c, c->gemm[fmt_index(f)][t], gemm_tiles(rows, gt.bm) * gemm_tiles(N, bn), 1, gt.threads(), 0,
                         args);
    }
    if (f != F_Q4) return fail(c, BRIK_EINVAL, "expert-grouped GEMM: q4 weights only");
    // blockIdx.y enumerates (expert, row tile) pairs: at most ceil(rows / BM) + E of them
    const void* p0b = pair ? pair->p0 : p0;
    const void* scb = pair ? pair->sc : sc;
    const void* mnb = pair ? pair->mn : mn;
    float* yb = pair ? pair->y : y;
    int mats = pair ? 2 : 1;
    void* args[] = {&xh, &rscale, &p0, &p1, &sc, &mn, &y, &Mi, &Ki, &Ni, &row_off, &Ei, &p0b, &scb, &mnb, &yb, &mats};
    // 1-D grid: (pairs rounded up to a multiple of 8) x column tiles x matrices; the kernel decodes the
    // index so that every block of one pair lands on one XCD
    const unsigned pairs = gemm_tiles(rows, gt.bm) + (unsigned)E;
    const unsigned blocks = (pairs + 7) / 8 * 8 * gemm_tiles(N, bn) * (unsigned)mats;
    // the 8-wave 64-row tile runs as its adaptive form (an expert tile of at most 32 live rows takes the
    // 32-row body): MoE down (K = 768, N = 2048) 28.4 -> 26.7 us kernel time. The 4-wave form measured
    // slower on gate + up in one launch (52.0 -> 54.9 us), its 32-row body being bound by the same
    // dequantization work per block, so that one runs as given; so does a forced tile.
    hipFunction_t fn = c->gemmg[t];
    if (c->opt_tile <= 0 && gt.bm == 64 && gt.tn == 1 && gt.pf == 1 && gt.nw == 8) fn = c->gemmg_adapt[1];
    return launch_fn(c, fn, blocks, 1, gt.threads(), 0, args);
}

// MFMA GEMM over `rows` activation rows: stage x as scaled f16 rows in the workspace, then run the
// tile kernel.
int gemm(brik_ctx* c, Fmt f, const float* x, const void* p0, const void* p1, const void* sc, const void* mn,
         float* y, int rows, int K, int N, const int* row_off, int E, const Scratch* fixed = nullptr,
         const WeightPair* pair = nullptr)
{
    if (K == 0) {                                           // empty sums
        if (pair) HIP_TRY_RC(fill_zero(c, pair->y, (size_t)rows * N));
        return fill_zero(c, y, (size_t)rows * N);
    }
    if (fixed) {
        // a fixed scratch holds the staged rows and, for split-K, the partial tiles after them: refuse
        // before anything is enqueued if they do not fit
        const size_t pb = splitk_part_bytes(c, f, rows, K, N, E);
        const size_t need = pb ? splitk_part_off(rows, K) + pb : 0;
        if (need > fixed->bytes)
            return fail(c, BRIK_EINVAL, "no-allocation call: needs %zu bytes of scratch (staged rows and split-K "
                        "partial tiles), the fixed buffer holds %zu", need, fixed->bytes);
    }
    long Kp;
    uint16_t* xh;
    float* rscale;
    HIP_TRY_RC(gemm_stage_ws(c, rows, K, Kp, xh, rscale, fixed));
    int Mi = rows, Ki = K, Kpi = (int)Kp;
    {
        void* args[] = {&x, &xh, &rscale, &Mi, &Ki, &Kpi};
        HIP_TRY_RC(launch(c, K_XPREP, xprep_grid(rows, Kp), 1, 256, 0, args));
    }
    return gemm_run(c, f, xh, rscale, p0, p1, sc, mn, y, rows, K, N, row_off, E, fixed, pair);
}

// GEMV variant for a launch over `rows` rows in total (one matrix or a plan's jobs) with shortest row
// K (index into kGemvVariants). `single`: one matrix at M = 1 (brik_matmul_t_*); `staged`: its blocks
// copy an x image staged once per call (a large single matrix) or by a GLU pair (a plan's consumer).
//
// Single matrices below the staged size: a launch of a few hundred blocks reaches HBM rate only when
// every block's loads go out at once, so the variant that gives at least ~256 blocks wins. Measured
// under graph replay on the Qwen3-4B shapes (us per launch): rows >= 4096 the whole-row 16-row blocks of
// variant 8 (q 4.37, gate 6.40 against 5.25 / 7.10 for the next best; q8 gate 9.01, q3 gate 6.63);
// fewer rows the 4-row blocks of variant 6, 64 lanes per row (k/v 3.46 against 4.07; wo K = 4096 5.05
// against 5.51; q8 k/v 3.44; q3 k/v 3.76); rows of K >= 8192 the 32-lane teams of variant 5 (down
// 8.52 against 8.99 with variant 6 and 9.74 with variant 8); q8 rows of K <= 1024 (the cfg 1 FFN shape
// K = 896: 28 groups, one step of 32 lanes) and q8 launches of 4096 rows or more the 8-row blocks of
// variant 10 (cfg 1 3.95 us against 4.13 with the 32-row blocks of variant 4; gate 8.13 against 8.99).
// Plans: large ones (the 36-layer set: 98k rows) stream whole rows per step with variant 7 (16 lanes x
// 5 groups = a K = 2560 row, 2 rows per team); the consumer of a GLU pair, which copies its image and
// so has no staging to amortize, takes the 4-row blocks of variant 6 (Qwen3-4B down, K = 9728: 640
// blocks, 6.74 us against 7.66 with variant 8); rows of K >= 8192 alone (a self-staged down
// projection) the one-row whole-row form of variant 8; rows of K >= 4096 (wo)
// variant 5; 8k-24k rows (a layer's gate/up) variant 0; 4k-8k rows (q/k/v) variant 1; smaller ones
// variant 8, which gives twice the blocks of variant 7.
// q3 large launches take variant 3 (4 rows per team share each staged x read) and the staged LM head
// variant 7 (42.8 us against 45 us with variant 3).
int gemv_variant(brik_ctx* c, Fmt f, long rows, int kmin, bool staged, bool single)
{
    if (c->opt_variant > 0) return c->opt_variant - 1;
    if (staged && !single) return 6;
    if (staged && f == F_Q3) return 7;
    if (single && rows < 96L * 256) {
        if (f == F_Q8 && kmin <= 1024 && rows < 32L * 256) return 10;
        if (kmin >= 8192) return 5;
        if (rows < 4096) return 6;
        return f == F_Q8 ? 10 : 8;
    }
    if (f == F_Q4) {
        if (rows >= 96L * 256) return 7;
        if (kmin >= 8192) return 8;
        if (kmin >= 4096) return 5;
        if (rows >= 32L * 256) return 0;
        return rows >= 16L * 256 ? 1 : 8;
    }
    if (f == F_Q3 && rows >= 96L * 256) return 3;
    if (f == F_Q8 && kmin <= 1024 && rows < 32L * 256) return 4;
    return rows >= 32L * 256 || kmin < 2048 ? 0 : 5;
}


// The sampling pre-work an LM head can run in its epilogue (brik_gemvh_*): the arguments of
// brik_topk_prep. `done` tells the caller whether the head ran it (else the caller runs the passes).
struct HeadArgs {
    float cap;
    int pen;
    float penalty;
    const int32_t* recent;
    int n_recent;
    uint32_t* maxima;
    bool done;
};

int matmul(brik_ctx* c, Fmt f, const float* x, const void* p0, const void* p1, const void* sc,
           const void* mn, float* y, int M, int K, int N, const Scratch* fixed = nullptr,
           HeadArgs* head = nullptr)
{
    c->last_path = 0;
    if (K == 0) return fill_zero(c, y, (size_t)M * N);   // empty sums, whatever the path
    // A large q4 / q3 matrix at M = 1 (an LM head) stages x once per call (brik_gemv_stage1_<fmt>, one
    // block) and its blocks copy the image instead of each staging x themselves. q8 measured no gain.
    const bool stage1 = M == 1 && N >= kPrestageRows && f != F_Q8 && c->opt_path != 2;
    // GEMV launch shape: one block per row set of RPI rows, capped; the block also stages its results
    const int v = gemv_variant(c, f, N, K, stage1, true);
    const int rpi = kGemvVariants[v].rpi();
    const unsigned sets = (unsigned)((N + rpi - 1) / rpi);
    // a launch that copies a staged image (stage1) runs 4 blocks per CU, each looping over its row sets
    // with the weight loads of the next set in flight (q3 LM head: 39.3 us against 41.2 us with one
    // block per row set)
    const unsigned cap = c->opt_gemv_blocks > 0 ? (unsigned)c->opt_gemv_blocks : stage1 ? 4 * kCUs : kGemvMaxBlocks;
    const unsigned gx = sets < cap ? sets : cap;
    const size_t lds = gemv_lds(K, f) + kGemvVariants[v].extra_lds((long)rpi * ((sets + gx - 1) / gx));
    const bool gemv_fits = lds <= kGemvMaxLds;
    // the MFMA GEMM reads scales in 16-group chunks, so a matrix of fewer than 16 groups (N * K < 512)
    // always takes the GEMV path (which handles any M)
    const bool tiny = (long)N * (K / kGroup) < 16;
    // a forced GEMM tile asks for the GEMM
    bool use_gemv = (M == 1 || tiny || (c->opt_tile == 0 && gemv_cheaper(f, M, K, N))) && gemv_fits;
    if (c->opt_path == 1) {
        if (!gemv_fits) return fail(c, BRIK_EINVAL, "forced GEMV: K=%d exceeds the LDS staging limit", K);
        use_gemv = true;
    } else if (c->opt_path == 2 && !tiny) {
        use_gemv = false;
    }
    int Ki = K, Ni = N;
    if (use_gemv) {
        const unsigned char* staged = nullptr;
        if (stage1) {
            void* img = nullptr;
            HIP_TRY_RC(take_scratch(c, fixed, c->sws, c->sws_bytes, (gemv_lds(K, f) + 15) & ~(size_t)15, img));
            staged = static_cast<const unsigned char*>(img);
            void* sargs[] = {&x, &Ki, &img};
            HIP_TRY_RC(launch(c, f == F_Q4 ? K_GEMV_STAGE1_Q4 : K_GEMV_STAGE1_Q3, 1, 1, kStageThreads, 0, sargs));
        }
        c->last_path = stage1 ? BRIK_PATH_GEMV_STAGED : BRIK_PATH_GEMV;
        if (head && stage1 && v == kHeadVariant) {
            // the LM head with the top-k pre-work in its epilogue: its LDS adds the row sums of a block
            // and a bitmap of its rows
            const long rows = (long)rpi * ((sets + gx - 1) / gx);
            const size_t hlds = lds + sizeof(float) * (size_t)rows + sizeof(uint32_t) * (size_t)((rows + 31) / 32);
            if (hlds <= kGemvMaxLds) {
                void* hargs[] = {&x, &p0, &p1, &sc, &mn, &y, &Ki, &Ni, &staged, &head->cap, &head->pen,
                                 &head->penalty, &head->recent, &head->n_recent, &head->maxima};
                head->done = true;
                return launch_fn(c, c->gemvh[fmt_index(f)], gx, 1, 256, hlds, hargs);
            }
        }
        void* args[] = {&x, &p0, &p1, &sc, &mn, &y, &Ki, &Ni, &staged};
        return launch_fn(c, c->gemv[fmt_index(f)][v], gx, (unsigned)M, 256, lds, args);
    }
    return gemm(c, f, x, p0, p1, sc, mn, y, M, K, N, nullptr, 0, fixed);
}

// ---- sampling pre-work -------------------------------------------------------------------------

constexpr int kTopkMax = 64;                      // BRIK_TOPK_MAX, TOPK_MAX in topk.hip
size_t topk_blocks(int n) { return ((size_t)n + 4095) / 4096; }          // 4 waves x 1024 logits
size_t topk_maxima(int n) { return 256 * topk_blocks(n); }                // one per lane (16 logits)
// workspace: lane maxima, then the LM-head logits
size_t topk_logits_off(int n) { return (4 * topk_maxima(n) + 255) / 256 * 256; }

int check_topk(brik_ctx* c, const char* who, int n, const int32_t* recent, int n_recent, float penalty, int k,
               const int32_t* ids, const float* vals, bool& pen)
{
    if (!c) return BRIK_EINVAL;
    if (n < 1) return fail(c, BRIK_EINVAL, "%s: n=%d must be >= 1", who, n);
    if (k < 1 || k > kTopkMax || k > n) return fail(c, BRIK_EINVAL, "%s: k=%d not in [1, min(64, n=%d)]", who, k, n);
    if (n_recent < 0) return fail(c, BRIK_EINVAL, "%s: n_recent=%d is negative", who, n_recent);
    // applied when the reference's `penalty && penalty !== 1 && recent.length` holds (kernels.ts:1947)
    pen = n_recent > 0 && penalty == penalty && penalty != 0.f && penalty != 1.f;
    if (pen && !recent) return fail(c, BRIK_EINVAL, "%s: recent is null", who);
    if (pen && !aligned(recent, 4)) return fail(c, BRIK_EALIGN, "%s: recent must be 4-byte aligned", who);
    if (!ids || !vals) return fail(c, BRIK_EINVAL, "%s: null output pointer", who);
    if (!aligned(ids, 4) || !aligned(vals, 4)) return fail(c, BRIK_EALIGN, "%s: outputs must be 4-byte aligned", who);
    return BRIK_OK;
}

// brik_topk_select over m lane maxima (one per 16 logits) in the top-k workspace.
int topk_select(brik_ctx* c, float* logits, int n, int m, int k, int32_t* ids, float* vals)
{
    uint32_t* maxima = static_cast<uint32_t*>(c->tws);
    void* args[] = {&logits, &n, &k, &maxima, &m, &ids, &vals};
    return launch(c, K_TOPK_SELECT, 1, 1, 1024, 0, args);
}

// The passes over a device logits vector (modified in place); the top-k workspace is ensured by the
// caller. Two launches: brik_topk_prep (softcap, penalty, lane maxima), brik_topk_select (one block:
// bound, candidates, sort, output).
int topk_passes(brik_ctx* c, float* logits, int n, const int32_t* recent, int n_recent, float penalty,
                float softcap, int k, int32_t* ids, float* vals, bool pen)
{
    uint32_t* maxima = static_cast<uint32_t*>(c->tws);
    int peni = pen ? 1 : 0;
    {
        void* args[] = {&logits, &n, &softcap, &recent, &n_recent, &penalty, &peni, &maxima};
        HIP_TRY_RC(launch(c, K_TOPK_PREP, (unsigned)topk_blocks(n), 1, 256, 0, args));
    }
    return topk_select(c, logits, n, (int)topk_maxima(n), k, ids, vals);
}

int ensure_topk_ws(brik_ctx* c, size_t bytes) { return ensure_buf(c, c->tws, c->tws_bytes, bytes); }

int lm_head_topk(brik_ctx* c, const char* who, Fmt f, const float* x, const void* p0, const void* p1,
                 const void* sc, const void* mn, int K, int vocab, const int32_t* recent, int n_recent,
                 float penalty, float softcap, int k, int32_t* ids, float* vals)
{
    bool pen = false;
    HIP_TRY_RC(check_topk(c, who, vocab, recent, n_recent, penalty, k, ids, vals, pen));
    if (K < 1) return fail(c, BRIK_EINVAL, "%s: K=%d must be >= 32", who, K);
    HIP_TRY_RC(ensure_topk_ws(c, topk_logits_off(vocab) + (size_t)vocab * 4));
    float* logits = reinterpret_cast<float*>(static_cast<char*>(c->tws) + topk_logits_off(vocab));
    HIP_TRY_RC(check_mm(c, who, x, p0, p1, sc, mn, logits, 1, K, vocab, f));
    // a q4 / q3 head staged once per call runs the pre-work in its epilogue (no pass over the logits);
    // any other takes the separate prep launch
    HeadArgs head{softcap, pen ? 1 : 0, penalty, recent, n_recent, static_cast<uint32_t*>(c->tws), false};
    HIP_TRY_RC(matmul(c, f, x, p0, p1, sc, mn, logits, 1, K, vocab, nullptr, &head));
    if (head.done) return topk_select(c, logits, vocab, (vocab + 15) / 16, k, ids, vals);
    return topk_passes(c, logits, vocab, recent, n_recent, penalty, softcap, k, ids, vals, pen);
}

// ---- self-validation (brik_self_validate) --------------------------------------------------------
// A CPU check inside the library, as the reference's engine carries one (selfValidate,
// src/lib/webgpu/kernels.ts:2255-2459): it runs the kernels on small seeded problems, downloads the
// planes the encoder produced and compares each result with an f64 sum over those planes' dequantized
// values. It never computes anything a caller receives.

uint64_t sv_next(uint64_t& s)
{
    uint64_t z = (s += 0x9E3779B97F4A7C15ull);
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

// uniform in [-1, 1), as the reference's rand() draws Math.random() * 2 - 1
float sv_unit(uint64_t& s) { return (float)((double)(sv_next(s) >> 11) * (1.0 / 9007199254740992.0) * 2.0 - 1.0); }

// IEEE half -> float (exact), for the downloaded scales and mins
double sv_f16(uint16_t h)
{
    const int e = (h >> 10) & 31, m = h & 1023;
    const double v = e == 0 ? std::ldexp((double)m, -24) : e == 31 ? (m ? NAN : INFINITY) : std::ldexp(1024.0 + m, e - 25);
    return (h & 0x8000) ? -v : v;
}

struct SvPlanes {
    size_t codes = 0, hi = 0, sc = 0, mn = 0, bytes = 0;   // byte offsets in one blob, and its size
};

SvPlanes sv_layout(Fmt f, size_t n)
{
    SvPlanes p;
    const size_t g = n / kGroup;
    const size_t cb = f == F_Q8 ? n : f == F_Q4 ? n / 2 : n / 4;
    p.codes = 0;
    p.hi = cb;
    p.sc = cb + (f == F_Q3 ? n / 8 : 0);
    p.mn = p.sc + 2 * g;
    p.bytes = p.mn + (f == F_Q8 ? 0 : 2 * g);
    return p;
}

// dequantized element i of a downloaded blob (the format's arithmetic: q * s, or q * s + m rounded
// once to f32, which is what the reference's dequantize produces)
float sv_deq(Fmt f, const std::vector<uint8_t>& b, const SvPlanes& p, size_t i)
{
    uint16_t sb, mb = 0;
    std::memcpy(&sb, &b[p.sc + 2 * (i / kGroup)], 2);
    if (f != F_Q8) std::memcpy(&mb, &b[p.mn + 2 * (i / kGroup)], 2);
    const double s = sv_f16(sb), m = sv_f16(mb);
    if (f == F_Q8) return (float)((double)(int8_t)b[p.codes + i] * s);
    uint32_t q;
    if (f == F_Q4) {
        q = (b[p.codes + i / 2] >> (4 * (i & 1))) & 15u;
    } else {
        uint32_t lw, hw;
        std::memcpy(&lw, &b[p.codes + 4 * (i / 16)], 4);
        std::memcpy(&hw, &b[p.hi + 4 * (i / 32)], 4);
        q = ((lw >> (2 * (i % 16))) & 3u) | (((hw >> (i % 32)) & 1u) << 2);
    }
    return (float)((double)q * s + m);
}

struct SvBuf {
    void* p = nullptr;
    ~SvBuf() { if (p) (void)hipFree(p); }
};

// One check; returns BRIK_OK, BRIK_EVALID (c->err names the failure) or a HIP / argument error.
int sv_case(brik_ctx* c, const char* stage, Fmt f, int M, int K, int N, bool moe, bool quant_check, bool relative,
            uint64_t seed)
{
    const size_t nw = (size_t)N * K;
    const int E = moe ? 4 : 1;
    const size_t nwe = nw * E;
    std::vector<float> W(nwe), A((size_t)M * K);
    for (auto& v : W) v = sv_unit(seed);
    for (auto& v : A) v = sv_unit(seed);
    const SvPlanes pl = sv_layout(f, nwe);
    SvBuf wf, blob, xa, ya, ro;
    HIP_TRY(c, hipSetDevice(c->device));
    HIP_TRY(c, hipMalloc(&wf.p, nwe * 4));
    HIP_TRY(c, hipMalloc(&blob.p, pl.bytes));
    HIP_TRY(c, hipMalloc(&xa.p, A.size() * 4));
    HIP_TRY(c, hipMalloc(&ya.p, (size_t)M * N * 4));
    HIP_TRY_RC(brik_h2d(c, wf.p, W.data(), nwe * 4));
    HIP_TRY_RC(brik_h2d(c, xa.p, A.data(), A.size() * 4));
    auto at = [&](size_t off) { return static_cast<char*>(blob.p) + off; };
    int r = f == F_Q8 ? brik_quantize_q8(c, (const float*)wf.p, (int8_t*)at(pl.codes), (uint16_t*)at(pl.sc), nwe)
          : f == F_Q4 ? brik_quantize_q4(c, (const float*)wf.p, (uint8_t*)at(pl.codes), (uint16_t*)at(pl.sc),
                                         (uint16_t*)at(pl.mn), nwe)
                      : brik_quantize_q3(c, (const float*)wf.p, (uint32_t*)at(pl.codes), (uint32_t*)at(pl.hi),
                                         (uint16_t*)at(pl.sc), (uint16_t*)at(pl.mn), nwe);
    HIP_TRY_RC(r);
    std::vector<uint8_t> hb(pl.bytes);
    HIP_TRY_RC(brik_d2h(c, hb.data(), blob.p, pl.bytes));
    if (quant_check) {
        // every dequantized weight within half a quantization step of the value it encodes, plus 2^-9
        // for the f16 rounding of the group's scale and min (at most (1 + range) 2^-11 with |w| < 1)
        for (size_t i = 0; i < nwe; ++i) {
            uint16_t sb;
            std::memcpy(&sb, &hb[pl.sc + 2 * (i / kGroup)], 2);
            const double d = std::fabs((double)sv_deq(f, hb, pl, i) - (double)W[i]);
            if (!(d <= 0.5 * sv_f16(sb) * (1.0 + 1e-3) + std::ldexp(1.0, -9)))
                return fail(c, BRIK_EVALID, "%s: element %zu dequantizes %g away from its input", stage, i, d);
        }
        return BRIK_OK;
    }
    std::vector<int32_t> off(E + 1);
    for (int e = 0; e <= E; ++e) off[e] = (int)((long)M * e / E);
    if (moe) {
        HIP_TRY(c, hipMalloc(&ro.p, off.size() * 4));
        HIP_TRY_RC(brik_h2d(c, ro.p, off.data(), off.size() * 4));
        r = brik_moe_matmul_t_q4(c, (const float*)xa.p, (const int32_t*)ro.p, (const uint8_t*)at(pl.codes),
                                 (const uint16_t*)at(pl.sc), (const uint16_t*)at(pl.mn), (float*)ya.p, E, M, K, N);
    } else if (f == F_Q8) {
        r = brik_matmul_t_q8(c, (const float*)xa.p, (const int8_t*)at(pl.codes), (const uint16_t*)at(pl.sc),
                             (float*)ya.p, M, K, N);
    } else if (f == F_Q4) {
        r = brik_matmul_t_q4(c, (const float*)xa.p, (const uint8_t*)at(pl.codes), (const uint16_t*)at(pl.sc),
                             (const uint16_t*)at(pl.mn), (float*)ya.p, M, K, N);
    } else {
        r = brik_matmul_t_q3(c, (const float*)xa.p, (const uint32_t*)at(pl.codes), (const uint32_t*)at(pl.hi),
                             (const uint16_t*)at(pl.sc), (const uint16_t*)at(pl.mn), (float*)ya.p, M, K, N);
    }
    HIP_TRY_RC(r);
    std::vector<float> got((size_t)M * N);
    HIP_TRY_RC(brik_d2h(c, got.data(), ya.p, got.size() * 4));
    std::vector<float> wd((size_t)N * K);
    for (int row = 0; row < M; ++row) {
        const int e = moe ? (int)(std::upper_bound(off.begin(), off.end(), row) - off.begin()) - 1 : 0;
        if (row == 0 || (moe && row == off[e]))
            for (size_t i = 0; i < nw; ++i) wd[i] = sv_deq(f, hb, pl, (size_t)e * nw + i);
        for (int col = 0; col < N; ++col) {
            double ref = 0, den = 0;
            for (int k = 0; k < K; ++k) {
                const double t = (double)A[(size_t)row * K + k] * (double)wd[(size_t)col * K + k];
                ref += t;
                den += std::fabs(t);
            }
            const double g = got[(size_t)row * N + col];
            const double tol = relative ? 1e-3 * den : 1e-3;
            if (!(std::fabs(g - (double)(float)ref) < tol))
                return fail(c, BRIK_EVALID, "%s: y[%d, %d] = %g, CPU reference %g", stage, row, col, g, (double)(float)ref);
        }
    }
    return BRIK_OK;
}

}  // namespace

extern "C" {

const char* brik_strerror(int code)
{
    switch (code) {
    case BRIK_EVALID: return "self-validation failed";
    case BRIK_OK: return "ok";
    case BRIK_EINVAL: return "invalid argument";
    case BRIK_EALIGN: return "misaligned pointer";
    case BRIK_EHIP: return "HIP runtime error";
    case BRIK_ENOMEM: return "out of device memory";
    case BRIK_ENODEV: return "no such device";
    case BRIK_EMODULE: return "code object load failed";
    default: return "unknown error";
    }
}

const char* brik_last_error(const brik_ctx* c) { return c ? c->err : "null context"; }

int brik_last_path(const brik_ctx* c) { return c ? c->last_path : 0; }

int brik_device_count(int* count)
{
    if (!count) return BRIK_EINVAL;
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess) n = 0;
    *count = n;
    return BRIK_OK;
}

int brik_create(int device, brik_ctx** out)
{
    if (!out) return BRIK_EINVAL;
    *out = nullptr;
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || device < 0 || device >= n) return BRIK_ENODEV;
    brik_ctx* c = new (std::nothrow) brik_ctx();
    if (!c) return BRIK_ENOMEM;
    c->device = device;
    auto bail = [&](int code) { brik_destroy(c); return code; };
    if (hipSetDevice(device) != hipSuccess) return bail(BRIK_ENODEV);
    hipDeviceProp_t prop;
    if (hipGetDeviceProperties(&prop, device) != hipSuccess) return bail(BRIK_ENODEV);
    if (std::strncmp(prop.gcnArchName, "gfx950", 6) != 0) return bail(BRIK_ENODEV);
    if (hipModuleLoadData(&c->module, brik_hsaco_begin) != hipSuccess) return bail(BRIK_EMODULE);
    for (int k = 0; k < K_COUNT; ++k)
        if (hipModuleGetFunction(&c->fn[k], c->module, kKernelNames[k]) != hipSuccess) return bail(BRIK_EMODULE);
    for (int f = 0; f < 3; ++f)
        for (int v = 0; v < kNumGemvVariants; ++v) {
            char name[64];
            const GemvVariant& gv = kGemvVariants[v];
            snprintf(name, sizeof name, "brik_gemv_%s_t%d_r%d_u%d_d%d", kFmtNames[f], gv.team, gv.r, gv.u, gv.d);
            if (hipModuleGetFunction(&c->gemv[f][v], c->module, name) != hipSuccess) return bail(BRIK_EMODULE);
            snprintf(name, sizeof name, "brik_gemvg_%s_t%d_r%d_u%d_d%d", kFmtNames[f], gv.team, gv.r, gv.u, gv.d);
            if (hipModuleGetFunction(&c->gemvg[f][v], c->module, name) != hipSuccess) return bail(BRIK_EMODULE);
        }
    for (int f = 1; f < 3; ++f) {
        char name[64];
        const GemvVariant& gv = kGluVariant;
        snprintf(name, sizeof name, "brik_gemvp_%s_t%d_r%d_u%d_d%d_n%d", kFmtNames[f], gv.team, gv.r, gv.u, gv.d,
                 kGluThreads);
        if (hipModuleGetFunction(&c->gemvp[f], c->module, name) != hipSuccess) return bail(BRIK_EMODULE);
        const GemvVariant& hv = kGemvVariants[kHeadVariant];
        snprintf(name, sizeof name, "brik_gemvh_%s_t%d_r%d_u%d_d%d", kFmtNames[f], hv.team, hv.r, hv.u, hv.d);
        if (hipModuleGetFunction(&c->gemvh[f], c->module, name) != hipSuccess) return bail(BRIK_EMODULE);
    }
    for (int f = 0; f < 3; ++f)
        for (int t = 0; t < kNumGemmTiles; ++t) {
            char name[64];
            char pf[16] = "";
            if (kGemmTiles[t].pf > 1) snprintf(pf, sizeof pf, "p%d", kGemmTiles[t].pf);
            snprintf(name, sizeof name, "brik_gemm_%s_%dx%d%s%s", kFmtNames[f], kGemmTiles[t].bm, kGemmTiles[t].tn,
                     kGemmTiles[t].nw == 8 ? "w8" : "", pf);
            if (hipModuleGetFunction(&c->gemm[f][t], c->module, name) != hipSuccess) return bail(BRIK_EMODULE);
            // the launch shape the runtime uses must fit the kernel's compiled bounds
            int max_threads = 0;
            if (hipFuncGetAttribute(&max_threads, HIP_FUNC_ATTRIBUTE_MAX_THREADS_PER_BLOCK, c->gemm[f][t]) != hipSuccess ||
                max_threads < (int)kGemmTiles[t].threads())
                return bail(BRIK_EMODULE);
            if (f != fmt_index(F_Q4)) continue;
            snprintf(name, sizeof name, "brik_gemmg_q4_%dx%d%s%s", kGemmTiles[t].bm, kGemmTiles[t].tn,
                     kGemmTiles[t].nw == 8 ? "w8" : "", pf);
            if (hipModuleGetFunction(&c->gemmg[t], c->module, name) != hipSuccess) return bail(BRIK_EMODULE);
            if (hipFuncGetAttribute(&max_threads, HIP_FUNC_ATTRIBUTE_MAX_THREADS_PER_BLOCK, c->gemmg[t]) != hipSuccess ||
                max_threads < (int)kGemmTiles[t].threads())
                return bail(BRIK_EMODULE);
        }
    if (hipModuleGetFunction(&c->gemmg_adapt[0], c->module, "brik_gemmg_q4_64a") != hipSuccess ||
        hipModuleGetFunction(&c->gemmg_adapt[1], c->module, "brik_gemmg_q4_64aw8") != hipSuccess)
        return bail(BRIK_EMODULE);
    for (int t = 0; t < kNumGemmTiles; ++t) {
        const GemmTile& g = kGemmTiles[t];
        if (g.tn != 1 || g.pf != 1) continue;
        char name[64];
        snprintf(name, sizeof name, "brik_gemm_f16_%dx1%s", g.bm, g.nw == 8 ? "w8" : "");
        if (hipModuleGetFunction(&c->gemm_f16[t], c->module, name) != hipSuccess) return bail(BRIK_EMODULE);
    }
    // the fixed scratch of brik_matmul_t_q4_noalloc, with this device current (once per device)
    c->scratch_err = brik_scratch_resolve(device, &c->scratch, &c->scratch_bytes);
    constexpr int kSkl[3] = {2, 4, 8};
    for (int f = 0; f < 3; ++f)
        for (int k = 0; k < 3; ++k) {
            char name[64];
            snprintf(name, sizeof name, "brik_gemm_sk_%s_k%d", kFmtNames[f], kSkl[k]);
            if (hipModuleGetFunction(&c->gemm_sk[f][k], c->module, name) != hipSuccess) return bail(BRIK_EMODULE);
        }
    if (hipStreamCreateWithFlags(&c->stream, hipStreamNonBlocking) != hipSuccess) return bail(BRIK_EHIP);
    if (hipEventCreate(&c->ev_begin) != hipSuccess || hipEventCreate(&c->ev_end) != hipSuccess)
        return bail(BRIK_EHIP);
    *out = c;
    return BRIK_OK;
}

void brik_destroy(brik_ctx* c)
{
    if (!c) return;
    // best-effort teardown: errors here have no caller to report to
    if (c->device >= 0) (void)hipSetDevice(c->device);
    if (c->stream && c->graph_capturing) {
        // a capture left open: end it (nothing recorded in it ran) so the stream can be synchronized
        hipGraph_t dropped = nullptr;
        if (hipStreamEndCapture(c->stream, &dropped) == hipSuccess && dropped) (void)hipGraphDestroy(dropped);
        c->graph_capturing = false;
    }
    if (c->stream) (void)hipStreamSynchronize(c->stream);
    for (const brik_ctx::Upload& u : c->ring_inflight) (void)hipEventDestroy(u.ev);
    for (hipEvent_t e : c->ring_events) (void)hipEventDestroy(e);
    if (c->ring) (void)hipHostFree(c->ring);
    if (c->ev_begin) (void)hipEventDestroy(c->ev_begin);
    if (c->ev_end) (void)hipEventDestroy(c->ev_end);
    if (c->stream) (void)hipStreamDestroy(c->stream);
    if (c->ws) (void)hipFree(c->ws);
    if (c->tws) (void)hipFree(c->tws);
    if (c->sws) (void)hipFree(c->sws);
    if (c->cws) (void)hipFree(c->cws);
    if (c->pws) (void)hipFree(c->pws);
    if (c->module) (void)hipModuleUnload(c->module);
    delete c;
}

int brik_alloc(brik_ctx* c, size_t bytes, void** dptr)
{
    if (c && c->graph_capturing) return fail(c, BRIK_EINVAL, "alloc / free: not allowed while a graph capture is open");
    if (!c || !dptr) return BRIK_EINVAL;
    *dptr = nullptr;
    HIP_TRY(c, hipSetDevice(c->device));
    HIP_TRY(c, hipMalloc(dptr, bytes ? bytes : 1));
    return BRIK_OK;
}

int brik_free(brik_ctx* c, void* dptr)
{
    if (c && c->graph_capturing) return fail(c, BRIK_EINVAL, "alloc / free: not allowed while a graph capture is open");
    if (!c) return BRIK_EINVAL;
    if (!dptr) return BRIK_OK;
    HIP_TRY(c, hipSetDevice(c->device));
    HIP_TRY(c, hipStreamSynchronize(c->stream));
    HIP_TRY(c, hipFree(dptr));
    return BRIK_OK;
}

static int copy(brik_ctx* c, void* dst, const void* src, size_t n, hipMemcpyKind kind)
{
    if (!c) return BRIK_EINVAL;
    if (n == 0) return BRIK_OK;
    if (!dst || !src) return fail(c, BRIK_EINVAL, "copy: null pointer");
    if (c->graph_capturing) return fail(c, BRIK_EINVAL, "copy: not allowed while a graph capture is open");
    HIP_TRY(c, hipSetDevice(c->device));
    HIP_TRY(c, hipMemcpyAsync(dst, src, n, kind, c->stream));
    HIP_TRY(c, hipStreamSynchronize(c->stream));
    return BRIK_OK;
}

int brik_h2d(brik_ctx* c, void* dst, const void* src, size_t n) { return copy(c, dst, src, n, hipMemcpyHostToDevice); }

int brik_h2d_async(brik_ctx* c, void* dst, const void* src, size_t n)
{
    if (!c) return BRIK_EINVAL;
    if (n == 0) return BRIK_OK;
    if (!dst || !src) return fail(c, BRIK_EINVAL, "h2d_async: null pointer");
    if (c->graph_capturing) return fail(c, BRIK_EINVAL, "copy: not allowed while a graph capture is open");
    constexpr size_t ring_bytes = BRIK_STAGING_RING_BYTES;
    if (n > ring_bytes / 2) return copy(c, dst, src, n, hipMemcpyHostToDevice);
    HIP_TRY(c, hipSetDevice(c->device));
    if (!c->ring) {
        HIP_TRY(c, hipHostMalloc(&c->ring, ring_bytes, hipHostMallocDefault));
    }
    // the slot: at the head, or at the start of the ring if it does not fit before the end
    size_t off = c->ring_head;
    if (off + n > ring_bytes) off = 0;
    // uploads still in flight that overlap [off, off + n): wait for the newest of them (events complete
    // in stream order, so every older upload has completed too) and retire them all up to it
    size_t last = 0;
    bool any = false;
    for (size_t i = 0; i < c->ring_inflight.size(); ++i) {
        const brik_ctx::Upload& u = c->ring_inflight[i];
        if (u.off < off + n && off < u.off + u.len) {
            last = i;
            any = true;
        }
    }
    if (any) {
        HIP_TRY(c, hipEventSynchronize(c->ring_inflight[last].ev));
        for (size_t i = 0; i <= last; ++i) {          // all complete
            c->ring_events.push_back(c->ring_inflight.front().ev);
            c->ring_inflight.pop_front();
        }
    }
    // retire uploads found complete at the front, without waiting
    while (!c->ring_inflight.empty() && hipEventQuery(c->ring_inflight.front().ev) == hipSuccess) {
        c->ring_events.push_back(c->ring_inflight.front().ev);
        c->ring_inflight.pop_front();
    }
    hipEvent_t ev = nullptr;
    if (!c->ring_events.empty()) {
        ev = c->ring_events.back();
        c->ring_events.pop_back();
    } else {
        HIP_TRY(c, hipEventCreateWithFlags(&ev, hipEventDisableTiming));
    }
    unsigned char* slot = static_cast<unsigned char*>(c->ring) + off;
    std::memcpy(slot, src, n);
    hipError_t e = hipMemcpyAsync(dst, slot, n, hipMemcpyHostToDevice, c->stream);
    if (e == hipSuccess) e = hipEventRecord(ev, c->stream);
    if (e != hipSuccess) {
        c->ring_events.push_back(ev);
        return fail(c, BRIK_EHIP, "h2d_async: %s", hipGetErrorString(e));
    }
    c->ring_inflight.push_back(brik_ctx::Upload{off, n, ev});
    c->ring_head = (off + n + 255) & ~(size_t)255;
    return BRIK_OK;
}
int brik_d2h(brik_ctx* c, void* dst, const void* src, size_t n) { return copy(c, dst, src, n, hipMemcpyDeviceToHost); }
int brik_d2d(brik_ctx* c, void* dst, const void* src, size_t n) { return copy(c, dst, src, n, hipMemcpyDeviceToDevice); }

int brik_sync(brik_ctx* c)
{
    if (c && c->graph_capturing) return fail(c, BRIK_EINVAL, "sync: not allowed while a graph capture is open");
    if (!c) return BRIK_EINVAL;
    HIP_TRY(c, hipSetDevice(c->device));
    HIP_TRY(c, hipStreamSynchronize(c->stream));
    return BRIK_OK;
}

int brik_matmul_t_q8(brik_ctx* c, const float* x, const int8_t* codes, const uint16_t* sc, float* y,
                     int M, int K, int N)
{
    int r = check_mm(c, "matmul_t_q8", x, codes, nullptr, sc, nullptr, y, M, K, N, F_Q8);
    if (r != BRIK_OK || M == 0 || N == 0) return r;
    return matmul(c, F_Q8, x, codes, nullptr, sc, nullptr, y, M, K, N);
}

int brik_matmul_t_q4(brik_ctx* c, const float* x, const uint8_t* nib, const uint16_t* sc,
                     const uint16_t* mn, float* y, int M, int K, int N)
{
    int r = check_mm(c, "matmul_t_q4", x, nib, nullptr, sc, mn, y, M, K, N, F_Q4);
    if (r != BRIK_OK || M == 0 || N == 0) return r;
    return matmul(c, F_Q4, x, nib, nullptr, sc, mn, y, M, K, N);
}

int brik_matmul_t_q4_noalloc(brik_ctx* c, const float* x, const uint8_t* nib, const uint16_t* sc,
                             const uint16_t* mn, float* y, int M, int K, int N)
{
    int r = check_mm(c, "matmul_t_q4_noalloc", x, nib, nullptr, sc, mn, y, M, K, N, F_Q4);
    if (r != BRIK_OK || M == 0 || N == 0) return r;
    if (!c->scratch)
        return fail(c, BRIK_EHIP, "matmul_t_q4_noalloc: the scratch array has no device address (%s)",
                    hipGetErrorString((hipError_t)c->scratch_err));
    const Scratch fixed{c->scratch, c->scratch_bytes};
    return matmul(c, F_Q4, x, nib, nullptr, sc, mn, y, M, K, N, &fixed);
}

int brik_matmul_t_q3(brik_ctx* c, const float* x, const uint32_t* lo, const uint32_t* hi,
                     const uint16_t* sc, const uint16_t* mn, float* y, int M, int K, int N)
{
    int r = check_mm(c, "matmul_t_q3", x, lo, hi, sc, mn, y, M, K, N, F_Q3);
    if (r != BRIK_OK || M == 0 || N == 0) return r;
    return matmul(c, F_Q3, x, lo, hi, sc, mn, y, M, K, N);
}

static int moe(brik_ctx* c, const char* who, const float* x, const int32_t* row_off, const uint8_t* nib,
               const uint16_t* sc, const uint16_t* mn, float* y, const WeightPair* pair, int E, int R, int K, int N)
{
    if (!c) return BRIK_EINVAL;
    c->last_path = 0;
    if (E < 0 || R < 0) return fail(c, BRIK_EINVAL, "%s: negative E=%d or R=%d", who, E, R);
    int r = check_mm(c, who, x, nib, nullptr, sc, mn, y, R, K, N, F_Q4);
    if (r == BRIK_OK && pair)
        r = check_mm(c, who, x, pair->p0, nullptr, pair->sc, pair->mn, pair->y, R, K, N, F_Q4);
    if (r != BRIK_OK || R == 0 || N == 0 || E == 0) return r;
    if (!row_off) return fail(c, BRIK_EINVAL, "%s: row_off is null", who);
    if (!aligned(row_off, 4)) return fail(c, BRIK_EALIGN, "%s: row_off must be 4-byte aligned", who);
    if (K == 0) return gemm(c, F_Q4, x, nib, nullptr, sc, mn, y, R, K, N, row_off, E, nullptr, pair);
    // the scale and min planes of all experts are addressed through one resource, in 16-group chunks
    const unsigned long long groups = (unsigned long long)E * N * (K / kGroup);
    if (groups < 16 || groups * 2 >= (1ull << 32))
        return fail(c, BRIK_EINVAL, "%s: E*N*K = %llu weight elements is outside [512, 2^35)", who,
                    groups * kGroup);
    return gemm(c, F_Q4, x, nib, nullptr, sc, mn, y, R, K, N, row_off, E, nullptr, pair);
}

int brik_moe_matmul_t_q4(brik_ctx* c, const float* x, const int32_t* row_off, const uint8_t* nib,
                         const uint16_t* sc, const uint16_t* mn, float* y, int E, int R, int K, int N)
{
    return moe(c, "moe_matmul_t_q4", x, row_off, nib, sc, mn, y, nullptr, E, R, K, N);
}

int brik_moe_matmul_t_q4_x2(brik_ctx* c, const float* x, const int32_t* row_off, const uint8_t* nib_a,
                            const uint16_t* sc_a, const uint16_t* mn_a, float* y_a, const uint8_t* nib_b,
                            const uint16_t* sc_b, const uint16_t* mn_b, float* y_b, int E, int R, int K, int N)
{
    const WeightPair pair{nib_b, sc_b, mn_b, y_b};
    return moe(c, "moe_matmul_t_q4_x2", x, row_off, nib_a, sc_a, mn_a, y_a, &pair, E, R, K, N);
}

static int dequant(brik_ctx* c, Kern k, const char* who, void** args, size_t n, const void* p0,
                   const void* out, size_t p0_align)
{
    if (!c) return BRIK_EINVAL;
    if (n % kGroup) return fail(c, BRIK_EINVAL, "%s: n=%zu is not a multiple of 32", who, n);
    if (n == 0) return BRIK_OK;
    if (!p0 || !out) return fail(c, BRIK_EINVAL, "%s: null pointer", who);
    if (!aligned(out, 16) || !aligned(p0, p0_align)) return fail(c, BRIK_EALIGN, "%s: misaligned pointer", who);
    const uint64_t n8 = n / 8;
    (void)n8;
    const unsigned gx = (unsigned)((n / 8 + 255) / 256);
    return launch(c, k, gx, 1, 256, 0, args);
}

int brik_dequant_q8_f32(brik_ctx* c, const int8_t* codes, const uint16_t* sc, float* out, size_t n)
{
    uint64_t n8 = n / 8;
    if (n && !sc) return fail(c, BRIK_EINVAL, "dequant_q8: null scales");
    void* args[] = {&codes, &sc, &out, &n8};
    return dequant(c, K_DEQ_Q8, "dequant_q8", args, n, codes, out, 8);
}

int brik_dequant_q4_f32(brik_ctx* c, const uint8_t* nib, const uint16_t* sc, const uint16_t* mn,
                        float* out, size_t n)
{
    uint64_t n8 = n / 8;
    if (n && (!sc || !mn)) return fail(c, BRIK_EINVAL, "dequant_q4: null scales/mins");
    void* args[] = {&nib, &sc, &mn, &out, &n8};
    return dequant(c, K_DEQ_Q4, "dequant_q4", args, n, nib, out, 4);
}

int brik_dequant_q3_f32(brik_ctx* c, const uint32_t* lo, const uint32_t* hi, const uint16_t* sc,
                        const uint16_t* mn, float* out, size_t n)
{
    uint64_t n8 = n / 8;
    if (n && (!hi || !sc || !mn)) return fail(c, BRIK_EINVAL, "dequant_q3: null plane");
    void* args[] = {&lo, &hi, &sc, &mn, &out, &n8};
    return dequant(c, K_DEQ_Q3, "dequant_q3", args, n, lo, out, 4);
}

// Encoders: two threads per 32-element group, 128 groups per block iteration; at most 2048 blocks (eight
// per CU, what their LDS allows), so each wave loops over several iterations and prefetches the next
// one's data.
static int quantize(brik_ctx* c, Kern k, const char* who, void** args, size_t n, const float* src,
                    const void* codes, const void* hi, const uint16_t* sc, const uint16_t* mn, bool asym)
{
    if (!c) return BRIK_EINVAL;
    if (n % kGroup) return fail(c, BRIK_EINVAL, "%s: n=%zu is not a multiple of 32", who, n);
    if (n == 0) return BRIK_OK;
    if (!src || !codes || !sc || (asym && !mn) || (k == K_QUANT_Q3 && !hi))
        return fail(c, BRIK_EINVAL, "%s: null pointer", who);
    if (!aligned(src, 16)) return fail(c, BRIK_EALIGN, "%s: src must be 16-byte aligned", who);
    if (!aligned(codes, 16) || (hi && !aligned(hi, 4)))
        return fail(c, BRIK_EALIGN, "%s: the code plane (q8 codes, q4 nibbles, q3 lo) must be 16-byte aligned, "
                    "the q3 hi plane 4-byte", who);
    if (!aligned(sc, 2) || (mn && !aligned(mn, 2)))
        return fail(c, BRIK_EALIGN, "%s: scales/mins must be 2-byte aligned", who);
    const size_t blocks = (n / kGroup + 127) / 128;
    return launch(c, k, (unsigned)(blocks < 2048 ? blocks : 2048), 1, 256, 0, args);
}

int brik_quantize_q8(brik_ctx* c, const float* src, int8_t* codes, uint16_t* sc, size_t n)
{
    size_t groups = n / kGroup;
    void* args[] = {&src, &codes, &sc, &groups};
    return quantize(c, K_QUANT_Q8, "quantize_q8", args, n, src, codes, nullptr, sc, nullptr, false);
}

int brik_quantize_q4(brik_ctx* c, const float* src, uint8_t* nib, uint16_t* sc, uint16_t* mn, size_t n)
{
    size_t groups = n / kGroup;
    void* args[] = {&src, &nib, &sc, &mn, &groups};
    return quantize(c, K_QUANT_Q4, "quantize_q4", args, n, src, nib, nullptr, sc, mn, true);
}

int brik_quantize_q3(brik_ctx* c, const float* src, uint32_t* lo, uint32_t* hi, uint16_t* sc, uint16_t* mn,
                     size_t n)
{
    size_t groups = n / kGroup;
    void* args[] = {&src, &lo, &hi, &sc, &mn, &groups};
    return quantize(c, K_QUANT_Q3, "quantize_q3", args, n, src, lo, hi, sc, mn, true);
}

// Convolution with a quantized weight: implicit MFMA GEMM when the weight rows are whole groups
// (K = Cin kh kw a multiple of 32) and the shape is large enough for the GEMM tiles, else the direct
// kernel. Option BRIK_OPT_PATH 1 forces the direct kernel, 2 the GEMM (when K % 32 == 0).
static int conv2d(brik_ctx* c, Fmt f, const char* who, const float* inp, const void* p0, const uint16_t* sc,
                  const uint16_t* mn, const float* bias, float* out, int Cin, int H, int W, int Cout, int kh, int kw,
                  int stride, int pad)
{
    if (!c) return BRIK_EINVAL;
    if (Cin < 1 || H < 1 || W < 1 || Cout < 1 || kh < 1 || kw < 1 || stride < 1 || pad < 0)
        return fail(c, BRIK_EINVAL, "%s: bad shape Cin=%d H=%d W=%d Cout=%d kernel %dx%d stride %d pad %d", who, Cin,
                    H, W, Cout, kh, kw, stride, pad);
    if (H + 2 * pad < kh || W + 2 * pad < kw)
        return fail(c, BRIK_EINVAL, "%s: the %dx%d kernel does not fit the padded %dx%d input", who, kh, kw, H, W);
    const int OH = (H + 2 * pad - kh) / stride + 1, OW = (W + 2 * pad - kw) / stride + 1;
    const long long K = (long long)Cin * kh * kw, M = (long long)OH * OW;
    const long long nw = K * Cout;
    if (nw % kGroup) return fail(c, BRIK_EINVAL, "%s: the weight has %lld elements, not a multiple of 32", who, nw);
    if (nw >= (1ll << 32) || M * Cout >= (1ll << 31) || (long long)Cin * H * W >= (1ll << 31))
        return fail(c, BRIK_EINVAL, "%s: tensor sizes exceed the 2^31-element limit", who);
    if (!inp || !p0 || !sc || (f == F_Q4 && !mn) || !out) return fail(c, BRIK_EINVAL, "%s: null pointer", who);
    if (!aligned(inp, 4) || !aligned(out, 16) || (bias && !aligned(bias, 4)) || !aligned(sc, 2) ||
        (mn && !aligned(mn, 2)) || !aligned(p0, 16))
        return fail(c, BRIK_EALIGN, "%s: inp / bias 4-byte, out and the code plane 16-byte, scales / mins 2-byte "
                    "aligned", who);
    // the GEMM's im2col staging addresses the input (and pad rows and columns before it) through a
    // 32-bit buffer offset: fewer than 2^29 elements
    const bool gemm_ok = K % kGroup == 0 && Cout * (K / kGroup) >= 16 && K <= (1 << 30) &&
                         (long long)Cin * H * W + (long long)pad * (W + 1) < (1ll << 29) && kh <= 64 && kw <= 64;
    bool use_gemm = gemm_ok && M >= 64;
    if (c->opt_path == 1) use_gemm = false;
    else if (c->opt_path == 2 && gemm_ok) use_gemm = true;
    int Ci = Cin, Hi = H, Wi = W, Co = Cout, khi = kh, kwi = kw, si = stride, pi = pad, OHi = OH, OWi = OW;
    if (!use_gemm) {
        // 256 output pixels x 16 output channels per block (conv.hip, conv_direct)
        const unsigned gx = (unsigned)((M + 255) / 256), gy = (unsigned)((Cout + 15) / 16);
        if (f == F_Q8) {
            void* args[] = {&inp, &p0, &sc, &bias, &out, &Ci, &Hi, &Wi, &Co, &khi, &kwi, &si, &pi, &OHi, &OWi};
            return launch(c, K_CONV_Q8, gx, gy, 256, 0, args);
        }
        void* args[] = {&inp, &p0, &sc, &mn, &bias, &out, &Ci, &Hi, &Wi, &Co, &khi, &kwi, &si, &pi, &OHi, &OWi};
        return launch(c, K_CONV_Q4, gx, gy, 256, 0, args);
    }
    const int rows = (int)M, Kint = (int)K;
    long Kp;
    uint16_t* xh;
    float* rscale;
    HIP_TRY_RC(gemm_stage_ws(c, rows, Kint, Kp, xh, rscale));
    // conv workspace: the GEMM output [M, Cout] (only without the fused epilogue), then the channel
    // maxima of the input [H W]
    const size_t yt_bytes = ((size_t)M * Cout * 4 + 255) & ~(size_t)255;
    // the GEMM writes out itself ([Cout, pixels] plus the bias) unless the split-K kernel runs it
    const bool fused = !use_splitk(c, f, rows, Kint, Cout, 0);
    HIP_TRY_RC(ensure_buf(c, c->cws, c->cws_bytes, (fused ? 0 : yt_bytes) + (size_t)H * W * 4));
    float* yt = static_cast<float*>(c->cws);
    float* cmax = reinterpret_cast<float*>(static_cast<unsigned char*>(c->cws) + (fused ? 0 : yt_bytes));
    int Kpi = (int)Kp, HW = H * W;
    {
        void* args[] = {&inp, &cmax, &Ci, &HW};
        HIP_TRY_RC(launch(c, K_CONV_CHANMAX, (unsigned)((HW + 31) / 32), 1, 1024, 0, args));
    }
    if (kh == 3 && kw == 3) {
        // 64 rows per block, 4 waves of 8 channels (9 chunks of 8 elements) each
        void* args[] = {&inp, &cmax, &xh, &rscale, (void*)&rows, (void*)&Kint, &Kpi, &Ci, &Hi, &Wi, &si, &pi, &OWi};
        HIP_TRY_RC(launch(c, K_XPREP_IM2COL3, (unsigned)((rows + 63) / 64), (unsigned)((Kp / 8 + 35) / 36), 256, 0,
                          args));
    } else {
        // 64 rows per block, 4 waves of 8 chunks of 8 elements each
        void* args[] = {&inp, &cmax, &xh, &rscale, (void*)&rows, (void*)&Kint, &Kpi, &Ci, &Hi, &Wi, &khi, &kwi, &si,
                        &pi, &OWi};
        HIP_TRY_RC(launch(c, K_XPREP_IM2COL, (unsigned)((rows + 63) / 64), (unsigned)((Kp / 8 + 31) / 32), 256, 0,
                          args));
    }
    if (fused) return gemm_run(c, f, xh, rscale, p0, nullptr, sc, mn, out, rows, Kint, Cout, nullptr, 0, nullptr, nullptr,
                               bias, 1);
    HIP_TRY_RC(gemm_run(c, f, xh, rscale, p0, nullptr, sc, mn, yt, rows, Kint, Cout, nullptr, 0));
    int P = rows;
    void* args[] = {&yt, &bias, &out, &P, &Co};
    return launch(c, K_CONV_OUT, (unsigned)((P + 31) / 32), (unsigned)((Cout + 31) / 32), 256, 0, args);
}

int brik_conv2d_q8(brik_ctx* c, const float* inp, const int8_t* codes, const uint16_t* sc, const float* bias,
                   float* out, int Cin, int H, int W, int Cout, int kh, int kw, int stride, int pad)
{
    return conv2d(c, F_Q8, "conv2d_q8", inp, codes, sc, nullptr, bias, out, Cin, H, W, Cout, kh, kw, stride, pad);
}

int brik_conv2d_q4(brik_ctx* c, const float* inp, const uint8_t* nib, const uint16_t* sc, const uint16_t* mn,
                   const float* bias, float* out, int Cin, int H, int W, int Cout, int kh, int kw, int stride, int pad)
{
    return conv2d(c, F_Q4, "conv2d_q4", inp, nib, sc, mn, bias, out, Cin, H, W, Cout, kh, kw, stride, pad);
}

// f16-weight matmul: the GEMV kernel for one activation row (x staged in LDS, K <= 16384) or for
// K % 8 != 0; otherwise staged f16 rows and the MFMA kernel. BRIK_OPT_PATH 1 / 2 force GEMV / MFMA.
int brik_matmul_t_f16w(brik_ctx* c, const float* x, const uint16_t* w, float* y, int M, int K, int N)
{
    if (!c) return BRIK_EINVAL;
    if (M < 0 || K < 0 || N < 0) return fail(c, BRIK_EINVAL, "matmul_t_f16w: negative shape M=%d K=%d N=%d", M, K, N);
    if (K % 4) return fail(c, BRIK_EINVAL, "matmul_t_f16w: K=%d is not a multiple of 4", K);
    if (M == 0 || N == 0) return BRIK_OK;
    if (!y) return fail(c, BRIK_EINVAL, "matmul_t_f16w: y is null");
    if (!aligned(y, 4)) return fail(c, BRIK_EALIGN, "matmul_t_f16w: y must be 4-byte aligned");
    if (K == 0) return fill_zero(c, y, (size_t)M * N);
    if (!x || !w) return fail(c, BRIK_EINVAL, "matmul_t_f16w: null operand pointer");
    if (!aligned(x, 16) || !aligned(w, 16))
        return fail(c, BRIK_EALIGN, "matmul_t_f16w: x and w must be 16-byte aligned");
    if ((long long)N * K >= (1ll << 31) || (long long)M * N >= (1ll << 31))
        return fail(c, BRIK_EINVAL, "matmul_t_f16w: tensors exceed 2^31 elements");
    const bool gemv_ok = K <= 16384, mfma_ok = K % 8 == 0;
    bool use_gemv = gemv_ok && (M == 1 || !mfma_ok);
    if (c->opt_path == 1 && gemv_ok) use_gemv = true;
    else if (c->opt_path == 2 && mfma_ok) use_gemv = false;
    if (!use_gemv && !mfma_ok)
        return fail(c, BRIK_EINVAL, "matmul_t_f16w: K=%d needs K %% 8 == 0 or K <= 16384", K);
    int Mi = M, Ki = K, Ni = N;
    if (use_gemv) {
        const long sets = ((long)N + 7) / 8;
        const unsigned gx = (unsigned)(sets < 16384 ? sets : 16384);
        void* args[] = {&x, &w, &y, &Ki, &Ni};
        return launch(c, K % 8 ? K_GEMV_F16W_V4 : K_GEMV_F16W_V8, gx, (unsigned)M, 256, (size_t)K * 4, args);
    }
    long Kp;
    uint16_t* xh;
    float* rscale;
    HIP_TRY_RC(gemm_stage_ws(c, M, K, Kp, xh, rscale));
    int Kpi = (int)Kp;
    {
        void* args[] = {&x, &xh, &rscale, &Mi, &Ki, &Kpi};
        HIP_TRY_RC(launch(c, K_XPREP, xprep_grid(M, Kp), 1, 256, 0, args));
    }
    if (K % kGroup == 0) {
        // the tiled MFMA GEMM with f16 weights (TN = 1 tiles): a forced tile, or the one of fewest
        // 256-CU rounds x tile area, as the quantized GEMM picks its dense tiles
        int best = -1;
        if (c->opt_tile > 0) {
            best = c->opt_tile - 1;
            if (!c->gemm_f16[best]) return fail(c, BRIK_EINVAL, "matmul_t_f16w: tile %d has no f16 form", c->opt_tile);
        } else {
            double best_cost = 0;
            for (int t = 0; t < kNumGemmTiles; ++t) {
                const GemmTile& g = kGemmTiles[t];
                if (!c->gemm_f16[t] || g.nw != 8) continue;
                const double rounds = std::ceil((double)gemm_tiles(M, g.bm) * gemm_tiles(N, g.bn()) / kCUs);
                const double penalty = g.bm == 128 ? 1.0 : g.bm == 96 ? 1.1 : g.bm == 64 ? 1.3 : 1.8;
                const double cost = rounds * g.bm * (double)g.bn() * penalty;
                if (best < 0 || cost < best_cost) {
                    best = t;
                    best_cost = cost;
                }
            }
        }
        const GemmTile& g = kGemmTiles[best];
        const void* none = nullptr;
        const int* no_rows = nullptr;
        int Ei = 0, trans = 0;
        const float* no_bias = nullptr;
        void* targs[] = {&xh, &rscale, &w, &none, &none, &none, &y, &Mi, &Ki, &Ni, &no_rows, &Ei, &no_bias, &trans};
        return launch_fn(c, c->gemm_f16[best], gemm_tiles(M, g.bm) * gemm_tiles(N, g.bn()), 1, g.threads(), 0,
                         targs);
    }
    // K % 32 != 0: the LDS-tiled kernel (K steps of 32 with zero-filled tails)
    void* args[] = {&xh, &rscale, &w, &y, &Mi, &Ki, &Ni, &Kpi};
    return launch(c, K_GEMM_F16W, (unsigned)((N + 127) / 128), (unsigned)((M + 63) / 64), 256, 0, args);
}

int brik_f16_to_f32(brik_ctx* c, const uint16_t* src, float* out, size_t n)
{
    if (!c) return BRIK_EINVAL;
    if (n == 0) return BRIK_OK;
    if (!src || !out) return fail(c, BRIK_EINVAL, "f16_to_f32: null pointer");
    if (!aligned(src, 16) || !aligned(out, 16)) return fail(c, BRIK_EALIGN, "f16_to_f32: src and out must be 16-byte aligned");
    const size_t blocks = ((n + 7) / 8 + 255) / 256;
    void* args[] = {&src, &out, &n};
    return launch(c, K_F16_TO_F32, (unsigned)(blocks < 8192 ? blocks : 8192), 1, 256, 0, args);
}

// The per-job checks of a plan (shapes, pointers, alignment, flags, LDS).
static int check_jobs(brik_ctx* c, Fmt f, const brik_gemv_job_ex* jobs, int njobs)
{
    for (int j = 0; j < njobs; ++j) {
        const brik_gemv_job& b = jobs[j].job;
        const brik_gemv_job_ex& e = jobs[j];
        if (e.flags & ~(BRIK_JOB_GAIN_ONE_PLUS | BRIK_JOB_ACT_GELU))
            return fail(c, BRIK_EINVAL, "gemv_plan: job %d has unknown flags 0x%x", j, (unsigned)e.flags);
        if ((e.gate && !aligned(e.gate, 16)) || (e.norm_w && !aligned(e.norm_w, 16)) || (e.res && !aligned(e.res, 4)))
            return fail(c, BRIK_EALIGN, "gemv_plan: job %d: gate / norm_w must be 16-byte, res 4-byte aligned", j);
        if (b.K < 32 || b.N < 1)
            return fail(c, BRIK_EINVAL, "gemv_plan: job %d has K=%d N=%d (need K >= 32, N >= 1)", j, b.K, b.N);
        int r = check_mm(c, "gemv_plan", b.x, b.p0, b.p1, b.scales, b.mins, b.y, 1, b.K, b.N, f);
        if (r != BRIK_OK) return r;
        if (gemv_lds(b.K, f) + kPlanPartialLds > kGemvMaxLds)
            return fail(c, BRIK_EINVAL, "gemv_plan: job %d K=%d exceeds the LDS staging limit", j, b.K);
    }
    return BRIK_OK;
}

// A grouped plan over `jobs`. With `image` (the consumer of a GLU pair: one job), the blocks copy that
// staged image of the job's input instead of staging it, and the plan holds a reference to it; with
// img_groups > 0 the producer writes only the image's first img_groups groups and the blocks stage the
// others themselves.
static int plan_create(brik_ctx* c, int fmt, const brik_gemv_job_ex* jobs, int njobs, brik_gemv_plan** out,
                       SharedBuf* image, int img_groups = 0)
{
    if (!c || !out) return BRIK_EINVAL;
    *out = nullptr;
    if (fmt != BRIK_FMT_Q8 && fmt != BRIK_FMT_Q4 && fmt != BRIK_FMT_Q3)
        return fail(c, BRIK_EINVAL, "gemv_plan: unknown format %d", fmt);
    if (njobs <= 0 || !jobs) return fail(c, BRIK_EINVAL, "gemv_plan: need at least one job");
    const Fmt f = Fmt(fmt);
    int r0 = check_jobs(c, f, jobs, njobs);
    if (r0 != BRIK_OK) return r0;
    int kmax = 0, kmin = 1 << 30;
    for (int j = 0; j < njobs; ++j) {
        kmax = jobs[j].job.K > kmax ? jobs[j].job.K : kmax;
        kmin = jobs[j].job.K < kmin ? jobs[j].job.K : kmin;
    }
    long rows = 0;
    for (int j = 0; j < njobs; ++j) rows += jobs[j].job.N;
    const int v = gemv_variant(c, f, rows, kmin, image != nullptr, false);
    const int rpi = kGemvVariants[v].rpi();
    // Blocks of about equal cost: rows per block ~ kPlanGroupRows / (K/32), in whole row sets of rpi
    // rows, at most kPlanMaxSets sets (bounded by the LDS partials buffer). A small plan (a decoder
    // layer's q/k/v or gate/up) would then have too few blocks to reach every CU's memory bandwidth:
    // the sets per block are halved until the launch has at least kPlanMinBlocks blocks (or one set
    // per block). Jobs are laid out in order of decreasing K, so the most expensive blocks are
    // dispatched first and the tail of the launch consists of the cheapest ones.
    std::vector<int> order(njobs);
    for (int j = 0; j < njobs; ++j) order[j] = j;
    std::stable_sort(order.begin(), order.end(), [&](int a, int b) { return jobs[a].job.K > jobs[b].job.K; });
    std::vector<brik_gemv_job_ex> sorted(njobs);
    std::vector<uint32_t> start(njobs + 1, 0), rpbs(njobs);
    std::vector<long> sets(njobs);
    const bool prestage = !image && (c->opt_plan_stage ? c->opt_plan_stage == 2 : rows >= kPrestageRows);
    // the lane partials of a block's row sets stay within the 16 KiB the per-job LDS check reserves
    long maxsets = (long)(kPlanPartialLds / kGemvVariants[v].extra_lds(rpi));
    const long capsets = prestage ? kPrestageMaxSets : kPlanMaxSets;
    maxsets = maxsets < 1 ? 1 : maxsets > capsets ? capsets : maxsets;
    const double group_rows = prestage ? kPrestageGroupRows : kPlanGroupRows;
    for (int k = 0; k < njobs; ++k) {
        const brik_gemv_job& b = jobs[order[k]].job;
        sorted[k] = jobs[order[k]];
        long s0 = lround(group_rows / ((double)(b.K / kGroup) * rpi));
        // a block that copies a staged image moves 112 B of it per group against 20 rpi B of q4 weights
        // per group and row set (17.5 %), so it takes at least two sets: the 36-layer q4 set's K = 9728
        // blocks (one set by the rule above) went 300.8-301.5 -> 299.3-300.0 us per step
        if (prestage && s0 < kPrestageMinSets) s0 = kPrestageMinSets;
        sets[k] = s0 < 1 ? 1 : s0 > maxsets ? maxsets : s0;
    }
    for (;;) {
        long blocks = 0, maxsets = 1;
        for (int k = 0; k < njobs; ++k) {
            blocks += (sorted[k].job.N + sets[k] * rpi - 1) / (sets[k] * rpi);
            maxsets = sets[k] > maxsets ? sets[k] : maxsets;
        }
        if (blocks >= kPlanMinBlocks || maxsets == 1) break;
        for (int k = 0; k < njobs; ++k) sets[k] = (sets[k] + 1) / 2;
    }
    long nblk = 0;
    for (int k = 0; k < njobs; ++k) nblk += (sorted[k].job.N + sets[k] * rpi - 1) / (sets[k] * rpi);
    if (prestage && nblk >= 8 * kPrestageTailBlocks) {   // plans of many blocks only: the tail stays short
        long tail = kPrestageTailBlocks;
        for (int k = njobs - 1; k >= 0 && tail > 0; --k) {
            sets[k] = 1;
            tail -= (sorted[k].job.N + rpi - 1) / rpi;
        }
    }
    if (c->opt_plan_sets > 0)
        for (int k = 0; k < njobs; ++k) sets[k] = c->opt_plan_sets < maxsets ? c->opt_plan_sets : maxsets;
    size_t lds = 0;
    for (int k = 0; k < njobs; ++k) {
        const brik_gemv_job& b = sorted[k].job;
        rpbs[k] = (uint32_t)(sets[k] * rpi);
        start[k + 1] = start[k] + (uint32_t)((b.N + rpbs[k] - 1) / rpbs[k]);
        const size_t need = gemv_lds(b.K, f) + kGemvVariants[v].extra_lds(rpbs[k]);
        lds = need > lds ? need : lds;
    }
    if (start[njobs] == 0 || start[njobs] > (1u << 31))
        return fail(c, BRIK_EINVAL, "gemv_plan: %u blocks is outside the launch range", start[njobs]);
    if (lds > kGemvMaxLds) return fail(c, BRIK_EINVAL, "gemv_plan: K=%d too large for LDS staging", kmax);
    // distinct input rows (x and the fused transform) and where each is staged
    std::vector<uint32_t> stage_off(njobs, 0);
    std::vector<brik_stage_input> inputs;
    size_t stage_bytes = 0;
    if (prestage) {
        for (int k = 0; k < njobs; ++k) {
            const brik_gemv_job_ex& e = sorted[k];
            int found = -1;
            for (size_t i = 0; i < inputs.size() && found < 0; ++i) {
                const brik_stage_input& in = inputs[i];
                if (in.x == e.job.x && in.gate == e.gate && in.norm_w == e.norm_w && in.K == e.job.K &&
                    in.flags == e.flags && std::memcmp(&in.eps, &e.eps, sizeof(float)) == 0)
                    found = (int)i;
            }
            if (found < 0) {
                inputs.push_back(brik_stage_input{e.job.x, e.gate, e.norm_w, e.eps, e.flags, e.job.K,
                                                  (uint32_t)stage_bytes});
                stage_bytes += (gemv_lds(e.job.K, f) + 15) & ~(size_t)15;
                found = (int)inputs.size() - 1;
                if (stage_bytes >= (1ull << 31)) return fail(c, BRIK_EINVAL, "gemv_plan: staged inputs exceed 2 GiB");
            }
            stage_off[k] = inputs[found].off;
        }
    }
    brik_gemv_plan* p = new (std::nothrow) brik_gemv_plan();
    if (!p) return BRIK_ENOMEM;
    // device tables: one brik_gemv_block per launch block (its job, rows and staged image), then the
    // staging pass's input table
    const size_t nblocks = start[njobs];
    const size_t inputs_off = sizeof(brik_gemv_block) * nblocks;
    const size_t bytes = inputs_off + sizeof(brik_stage_input) * inputs.size();
    std::vector<unsigned char> host(bytes, 0);
    brik_gemv_block* bt = reinterpret_cast<brik_gemv_block*>(host.data());
    for (int k = 0; k < njobs; ++k) {
        for (uint32_t b = start[k]; b < start[k + 1]; ++b) {
            brik_gemv_block& d = bt[b];
            d.job = sorted[k];
            d.r0 = (int32_t)((b - start[k]) * rpbs[k]);
            d.r1 = std::min(sorted[k].job.N, d.r0 + (int32_t)rpbs[k]);
            d.stage_off = stage_off[k];
            d.img_groups = image ? (uint32_t)img_groups : 0u;
        }
    }
    if (!inputs.empty()) std::memcpy(host.data() + inputs_off, inputs.data(), sizeof(brik_stage_input) * inputs.size());
    int r = brik_alloc(c, bytes, &p->dev);
    if (r == BRIK_OK) r = brik_h2d(c, p->dev, host.data(), bytes);
    if (r == BRIK_OK && prestage) r = brik_alloc(c, stage_bytes, &p->stage);
    if (r != BRIK_OK) { brik_free(c, p->dev); brik_free(c, p->stage); delete p; return r; }
    if (prestage) {
        p->stager = c->fn[f == F_Q8 ? K_GEMV_STAGE_Q8 : f == F_Q4 ? K_GEMV_STAGE_Q4 : K_GEMV_STAGE_Q3];
        p->ninputs = (int)inputs.size();
        p->inputs_off = inputs_off;
    }
    if (image) {
        p->stage = image->ptr;
        p->image = image;
        ++image->refs;
    }
    p->kernel = c->gemvg[fmt_index(f)][v];
    p->njobs = njobs;
    p->blocks = start[njobs];
    p->lds = lds;
    *out = p;
    return BRIK_OK;
}

int brik_gemv_plan_create_ex(brik_ctx* c, int fmt, const brik_gemv_job_ex* jobs, int njobs, brik_gemv_plan** out)
{
    return plan_create(c, fmt, jobs, njobs, out, nullptr);
}

int brik_gemv_plan_create_glu(brik_ctx* c, int fmt, const brik_gemv_job_ex* gate, const brik_gemv_job_ex* up,
                              const brik_gemv_job_ex* down, brik_gemv_plan** gate_up, brik_gemv_plan** down_plan)
{
    if (!c || !gate_up || !down_plan) return BRIK_EINVAL;
    *gate_up = nullptr;
    *down_plan = nullptr;
    if (fmt != BRIK_FMT_Q8 && fmt != BRIK_FMT_Q4 && fmt != BRIK_FMT_Q3)
        return fail(c, BRIK_EINVAL, "gemv_plan_glu: unknown format %d", fmt);
    if (!gate || !up || !down) return fail(c, BRIK_EINVAL, "gemv_plan_glu: gate, up and down jobs are required");
    const brik_gemv_job &g = gate->job, &u = up->job, &d = down->job;
    if (g.x != u.x || g.K != u.K || g.N != u.N || gate->gate != up->gate || gate->norm_w != up->norm_w ||
        gate->flags != up->flags || std::memcmp(&gate->eps, &up->eps, sizeof(float)) != 0)
        return fail(c, BRIK_EINVAL, "gemv_plan_glu: gate and up must share x, K, N and the input fusion");
    if (g.y == u.y) return fail(c, BRIK_EINVAL, "gemv_plan_glu: gate and up need distinct outputs");
    if (d.K != g.N || d.x != u.y || down->gate != g.y)
        return fail(c, BRIK_EINVAL,
                    "gemv_plan_glu: down must multiply act(gate.y) * up.y (down.gate = gate.y, down.x = up.y, "
                    "down.K = gate.N)");
    if (down->norm_w || (down->flags & ~BRIK_JOB_ACT_GELU))
        return fail(c, BRIK_EINVAL, "gemv_plan_glu: down takes no RMSNorm (flags: BRIK_JOB_ACT_GELU only)");
    const brik_gemv_job_ex both[2] = {*gate, *up};
    if (fmt == BRIK_FMT_Q8) {
        // no q8 pair kernel: the two ordinary plans (down stages its own input)
        int r = brik_gemv_plan_create_ex(c, fmt, both, 2, gate_up);
        if (r != BRIK_OK) return r;
        r = brik_gemv_plan_create_ex(c, fmt, down, 1, down_plan);
        if (r != BRIK_OK) {
            brik_gemv_plan_destroy(c, *gate_up);
            *gate_up = nullptr;
        }
        return r;
    }
    const Fmt f = Fmt(fmt);
    int r = check_jobs(c, f, both, 2);
    if (r == BRIK_OK) r = check_jobs(c, f, down, 1);
    if (r != BRIK_OK) return r;
    // The launch's blocks of whole groups (32 rows of each matrix, 8 waves) are equal units: with
    // 9728 rows (304 groups) on 256 CUs, 48 CUs ran two of them while the others ran one (12.0 us
    // against 9.7 us for the unlinked gate/up plan). When the groups exceed a whole number of rounds
    // of CUs by at most half a round, the remainder runs in blocks of 8 rows of each matrix that write
    // act(gate) * up of their rows after the image, and the consumer stages those groups itself (the
    // same code on the same values as its own staging, so its input stays bit-identical).
    const int groups = g.N / kGroup;
    const int rem = groups % (int)kCUs;
    const int nfull = groups > (int)kCUs && rem > 0 && rem <= (int)kCUs / 2 ? groups - rem : groups;
    // the image of down's input: zero groups (group G stays the zero group), then the flag -1 (read the
    // groups' own markers) and the RMSNorm factor 1; then the values of the groups past nfull
    const size_t ib = (gemv_lds(d.K, f) + 15) & ~(size_t)15;
    const size_t tail_bytes = sizeof(float) * kGroup * (size_t)(groups - nfull);
    std::vector<unsigned char> host(ib, 0);
    const size_t tail = (size_t)112 * (d.K / kGroup + 1);
    const int32_t scan = -1;
    const float one = 1.f;
    std::memcpy(host.data() + tail, &scan, sizeof scan);
    std::memcpy(host.data() + tail + 4, &one, sizeof one);
    SharedBuf* img = new (std::nothrow) SharedBuf();
    brik_gemv_plan* p = new (std::nothrow) brik_gemv_plan();
    if (!img || !p) {
        delete img;
        delete p;
        return BRIK_ENOMEM;
    }
    r = brik_alloc(c, ib + tail_bytes, &img->ptr);
    if (r == BRIK_OK) r = brik_h2d(c, img->ptr, host.data(), ib);
    if (r == BRIK_OK) r = brik_alloc(c, sizeof both, &p->dev);
    if (r == BRIK_OK) r = brik_h2d(c, p->dev, both, sizeof both);
    if (r != BRIK_OK) {
        brik_free(c, img->ptr);
        brik_free(c, p->dev);
        delete img;
        delete p;
        return r;
    }
    p->glu = true;
    p->kernel = c->gemvp[fmt_index(f)];
    p->njobs = 2;
    p->glu_full = nfull;
    p->blocks = (unsigned)(nfull + (groups - nfull) * (kGroup / kGluTailRows));
    p->lds = gemv_lds(g.K, f) + kGluVariant.extra_lds(2 * kGluRows);
    p->act_flags = down->flags & BRIK_JOB_ACT_GELU;
    p->stage = img->ptr;
    p->image = img;
    img->refs = 1;
    r = plan_create(c, fmt, down, 1, down_plan, img, nfull < groups ? nfull : 0);
    if (r != BRIK_OK) {
        brik_gemv_plan_destroy(c, p);
        return r;
    }
    *gate_up = p;
    return BRIK_OK;
}

int brik_gemv_plan_create(brik_ctx* c, int fmt, const brik_gemv_job* jobs, int njobs, brik_gemv_plan** out)
{
    if (!c || !out) return BRIK_EINVAL;
    if (njobs <= 0 || !jobs) return fail(c, BRIK_EINVAL, "gemv_plan: need at least one job");
    std::vector<brik_gemv_job_ex> ex(njobs);
    for (int j = 0; j < njobs; ++j) ex[j] = brik_gemv_job_ex{jobs[j], nullptr, nullptr, nullptr, 0.f, 0};
    return brik_gemv_plan_create_ex(c, fmt, ex.data(), njobs, out);
}

int brik_gemv_plan_run(brik_ctx* c, const brik_gemv_plan* p)
{
    if (!c || !p) return BRIK_EINVAL;
    if (p->glu) {
        const brik_gemv_job_ex* jobs = (const brik_gemv_job_ex*)p->dev;
        void* img = p->stage;
        int af = p->act_flags;
        int nfull = p->glu_full;
        void* args[] = {&jobs, &img, &af, &nfull};
        return launch_fn(c, p->kernel, p->blocks, 1, kGluThreads, p->lds, args);
    }
    const brik_gemv_block* blocks = static_cast<const brik_gemv_block*>(p->dev);
    const unsigned char* stage = static_cast<const unsigned char*>(p->stage);
    if (p->stager) {
        // one block per distinct input row; the GEMV launch that follows on the stream reads the images
        const brik_stage_input* inputs =
            reinterpret_cast<const brik_stage_input*>(static_cast<const unsigned char*>(p->dev) + p->inputs_off);
        void* stage_buf = p->stage;
        void* sargs[] = {&inputs, &stage_buf};
        HIP_TRY_RC(launch_fn(c, p->stager, (unsigned)p->ninputs, 1, kStageThreads, 0, sargs));
    }
    void* args[] = {&blocks, &stage};
    return launch_fn(c, p->kernel, p->blocks, 1, 256, p->lds, args);
}

void brik_gemv_plan_destroy(brik_ctx* c, brik_gemv_plan* p)
{
    if (!p) return;
    if (c) {
        brik_free(c, p->dev);
        if (!p->image) brik_free(c, p->stage);
    }
    if (p->image && --p->image->refs == 0) {
        if (c) brik_free(c, p->image->ptr);
        delete p->image;
    }
    delete p;
}

int brik_logits_topk(brik_ctx* c, float* logits, int n, const int32_t* recent, int n_recent, float penalty,
                     float softcap, int k, int32_t* out_ids, float* out_vals)
{
    bool pen = false;
    HIP_TRY_RC(check_topk(c, "logits_topk", n, recent, n_recent, penalty, k, out_ids, out_vals, pen));
    if (!logits) return fail(c, BRIK_EINVAL, "logits_topk: logits is null");
    if (!aligned(logits, 4)) return fail(c, BRIK_EALIGN, "logits_topk: logits must be 4-byte aligned");
    HIP_TRY_RC(ensure_topk_ws(c, topk_logits_off(n)));
    return topk_passes(c, logits, n, recent, n_recent, penalty, softcap, k, out_ids, out_vals, pen);
}

int brik_lm_head_topk_q8(brik_ctx* c, const float* x, const int8_t* codes, const uint16_t* sc, int K, int vocab,
                         const int32_t* recent, int n_recent, float penalty, float softcap, int k, int32_t* out_ids,
                         float* out_vals)
{
    return lm_head_topk(c, "lm_head_topk_q8", F_Q8, x, codes, nullptr, sc, nullptr, K, vocab, recent, n_recent,
                        penalty, softcap, k, out_ids, out_vals);
}

int brik_lm_head_topk_q4(brik_ctx* c, const float* x, const uint8_t* nib, const uint16_t* sc, const uint16_t* mn,
                         int K, int vocab, const int32_t* recent, int n_recent, float penalty, float softcap, int k,
                         int32_t* out_ids, float* out_vals)
{
    return lm_head_topk(c, "lm_head_topk_q4", F_Q4, x, nib, nullptr, sc, mn, K, vocab, recent, n_recent, penalty,
                        softcap, k, out_ids, out_vals);
}

int brik_lm_head_topk_q3(brik_ctx* c, const float* x, const uint32_t* lo, const uint32_t* hi, const uint16_t* sc,
                         const uint16_t* mn, int K, int vocab, const int32_t* recent, int n_recent, float penalty,
                         float softcap, int k, int32_t* out_ids, float* out_vals)
{
    return lm_head_topk(c, "lm_head_topk_q3", F_Q3, x, lo, hi, sc, mn, K, vocab, recent, n_recent, penalty,
                        softcap, k, out_ids, out_vals);
}

int brik_graph_begin(brik_ctx* c)
{
    if (!c) return BRIK_EINVAL;
    if (c->graph_capturing) return fail(c, BRIK_EINVAL, "graph_begin: a capture is already open");
    HIP_TRY(c, hipSetDevice(c->device));
    HIP_TRY(c, hipStreamBeginCapture(c->stream, hipStreamCaptureModeThreadLocal));
    c->graph_capturing = true;
    c->graph_used_ws = false;
    return BRIK_OK;
}

int brik_graph_end(brik_ctx* c, brik_graph** out)
{
    if (!c || !out) return BRIK_EINVAL;
    *out = nullptr;
    if (!c->graph_capturing) return fail(c, BRIK_EINVAL, "graph_end: no capture is open");
    c->graph_capturing = false;
    brik_graph* g = new (std::nothrow) brik_graph();
    if (!g) {
        // close the capture all the same, so the stream works again
        hipGraph_t dropped = nullptr;
        if (hipStreamEndCapture(c->stream, &dropped) == hipSuccess && dropped) (void)hipGraphDestroy(dropped);
        return BRIK_ENOMEM;
    }
    hipError_t e = hipStreamEndCapture(c->stream, &g->graph);
    if (e == hipSuccess) e = hipGraphInstantiate(&g->exec, g->graph, nullptr, nullptr, 0);
    if (e != hipSuccess) {
        if (g->graph) (void)hipGraphDestroy(g->graph);
        delete g;
        return fail(c, BRIK_EHIP, "graph_end: %s", hipGetErrorString(e));
    }
    g->ws_generation = c->ws_generation;
    g->uses_ws = c->graph_used_ws;
    *out = g;
    return BRIK_OK;
}

int brik_graph_launch(brik_ctx* c, const brik_graph* g)
{
    if (!c || !g) return BRIK_EINVAL;
    if (g->uses_ws && g->ws_generation != c->ws_generation)
        return fail(c, BRIK_EINVAL, "graph_launch: a context workspace was reallocated after this graph was "
                                    "recorded (a larger call ran since); record the graph again");
    HIP_TRY(c, hipSetDevice(c->device));
    HIP_TRY(c, hipGraphLaunch(g->exec, c->stream));
    return BRIK_OK;
}

void brik_graph_destroy(brik_ctx* c, brik_graph* g)
{
    (void)c;
    if (!g) return;
    if (g->exec) (void)hipGraphExecDestroy(g->exec);
    if (g->graph) (void)hipGraphDestroy(g->graph);
    delete g;
}

int brik_timer_begin(brik_ctx* c)
{
    if (!c) return BRIK_EINVAL;
    HIP_TRY(c, hipSetDevice(c->device));
    HIP_TRY(c, hipEventRecord(c->ev_begin, c->stream));
    return BRIK_OK;
}

int brik_timer_end(brik_ctx* c, float* ms)
{
    if (!c || !ms) return BRIK_EINVAL;
    HIP_TRY(c, hipSetDevice(c->device));
    HIP_TRY(c, hipEventRecord(c->ev_end, c->stream));
    HIP_TRY(c, hipEventSynchronize(c->ev_end));
    HIP_TRY(c, hipEventElapsedTime(ms, c->ev_begin, c->ev_end));
    return BRIK_OK;
}

int brik_fence_record(brik_ctx* c, brik_fence** out)
{
    if (!c || !out) return BRIK_EINVAL;
    *out = nullptr;
    if (c->graph_capturing) return fail(c, BRIK_EINVAL, "fence: not allowed while a graph capture is open");
    brik_fence* f = new (std::nothrow) brik_fence();
    if (!f) return BRIK_ENOMEM;
    f->device = c->device;
    hipError_t e = hipSetDevice(c->device);
    if (e == hipSuccess) e = hipEventCreateWithFlags(&f->ev, hipEventDisableTiming);
    if (e == hipSuccess) e = hipEventRecord(f->ev, c->stream);
    if (e != hipSuccess) {
        brik_fence_destroy(f);
        return fail(c, BRIK_EHIP, "fence: %s", hipGetErrorString(e));
    }
    *out = f;
    return BRIK_OK;
}

int brik_fence_d2h(brik_fence* f, void* dst, const void* src, size_t bytes)
{
    if (!f) return BRIK_EINVAL;
    if (bytes && (!dst || !src)) {
        snprintf(f->err, sizeof f->err, "fence_d2h: null pointer");
        return BRIK_EINVAL;
    }
    hipError_t e = hipSetDevice(f->device);
    if (e == hipSuccess) e = hipEventSynchronize(f->ev);
    // the context stream is non-blocking, so this copy on the null stream waits for nothing else
    if (e == hipSuccess && bytes) e = hipMemcpy(dst, src, bytes, hipMemcpyDeviceToHost);
    if (e != hipSuccess) {
        snprintf(f->err, sizeof f->err, "fence_d2h: %s", hipGetErrorString(e));
        return BRIK_EHIP;
    }
    return BRIK_OK;
}

const char* brik_fence_error(const brik_fence* f) { return f ? f->err : "null fence"; }

void brik_fence_destroy(brik_fence* f)
{
    if (!f) return;
    if (f->ev) {
        (void)hipSetDevice(f->device);
        (void)hipEventDestroy(f->ev);
    }
    delete f;
}

int brik_self_validate(brik_ctx* c, char* stage, size_t cap)
{
    if (!c) return BRIK_EINVAL;
    if (stage && cap) stage[0] = 0;
    if (c->graph_capturing) return fail(c, BRIK_EINVAL, "self_validate: not allowed while a graph capture is open");
    struct Check {
        const char* stage;
        Fmt f;
        int M, K, N;
        bool moe, quant, relative;
    };
    // the reference's quantized checks in its order (kernels.ts:2325-2459), then two of this library's
    const Check checks[] = {
        {"matmulQ4", F_Q4, 1, 128, 6, false, false, false},
        {"quantize_q4", F_Q4, 1, 128, 6, false, true, false},
        {"matmulQ3", F_Q3, 5, 128, 6, false, false, false},
        {"matmul_q4_tiled", F_Q4, 5, 128, 6, false, false, false},
        {"matmul_q4_shared", F_Q4, 20, 128, 18, false, false, false},
        {"matmulQ8", F_Q8, 1, 128, 6, false, false, false},
        {"quantize_q8", F_Q8, 1, 128, 6, false, true, false},
        {"matmul_q8_tiled", F_Q8, 5, 128, 6, false, false, false},
        {"matmul_q8_shared", F_Q8, 20, 128, 18, false, false, false},
        {"matmul_q4_prefill", F_Q4, 40, 1024, 256, false, false, true},
        {"moe_matmul_q4", F_Q4, 40, 512, 96, true, false, true},
    };
    uint64_t seed = 0x5EEDB41Cull;
    for (const Check& k : checks) {
        const int r = sv_case(c, k.stage, k.f, k.M, k.K, k.N, k.moe, k.quant, k.relative, seed);
        seed += 0x1000;
        if (r != BRIK_OK) {
            if (stage && cap) snprintf(stage, cap, "%s", k.stage);
            return r;
        }
    }
    return BRIK_OK;
}

int brik_set_option(brik_ctx* c, int key, int value)
{
    if (!c) return BRIK_EINVAL;
    switch (key) {
    case BRIK_OPT_PATH:
        if (value < 0 || value > 2) return fail(c, BRIK_EINVAL, "BRIK_OPT_PATH: %d not in 0..2", value);
        c->opt_path = value;
        return BRIK_OK;
    case BRIK_OPT_GEMV_VARIANT:
        if (value < 0 || value > kNumGemvVariants)
            return fail(c, BRIK_EINVAL, "BRIK_OPT_GEMV_VARIANT: %d not in 0..%d", value, kNumGemvVariants);
        c->opt_variant = value;
        return BRIK_OK;
    case BRIK_OPT_GEMM_TILE:
        if (value < 0 || value > kNumGemmTiles)
            return fail(c, BRIK_EINVAL, "BRIK_OPT_GEMM_TILE: %d not in 0..%d", value, kNumGemmTiles);
        c->opt_tile = value;
        return BRIK_OK;
    case BRIK_OPT_PLAN_STAGE:
        if (value < 0 || value > 2) return fail(c, BRIK_EINVAL, "BRIK_OPT_PLAN_STAGE: %d not in 0..2", value);
        c->opt_plan_stage = value;
        return BRIK_OK;
    case BRIK_OPT_SPLITK:
        if (value < 0 || value > 2) return fail(c, BRIK_EINVAL, "BRIK_OPT_SPLITK: %d not in 0..2", value);
        c->opt_splitk = value;
        return BRIK_OK;
    case BRIK_OPT_PLAN_SETS:
        if (value < 0 || value > 64) return fail(c, BRIK_EINVAL, "BRIK_OPT_PLAN_SETS: %d not in 0..64", value);
        c->opt_plan_sets = value;
        return BRIK_OK;
    case BRIK_OPT_GEMV_BLOCKS:
        if (value < 0 || value > (int)kGemvMaxBlocks)
            return fail(c, BRIK_EINVAL, "BRIK_OPT_GEMV_BLOCKS: %d not in 0..%u", value, kGemvMaxBlocks);
        c->opt_gemv_blocks = value;
        return BRIK_OK;
    default:
        return fail(c, BRIK_EINVAL, "unknown option %d", key);
    }
}

}  // extern "C"
