// Sampling pre-work on a logits vector, the passes decodeTopKQ8 records after the LM head
// (src/lib/webgpu/kernels.ts:1940-1958; shaders softcap_logits / penalize_logits / top_k,
// src/lib/webgpu/shaders.ts:954-1020), in the same order and, like the reference, in place:
//   1. softcap (cap > 0):     l = cap * tanh(l / cap)                         (shaders.ts:954-964)
//   2. repetition penalty:    l = l > 0 ? l / p : l * p  for each recent id   (shaders.ts:966-980)
//   3. top-k (k <= 64):       the k largest logits, ids and values sorted descending (shaders.ts:982-1020)
// The reference's top_k runs in one 128-thread workgroup and is exact unless more than 8 of the true
// top-k share an id mod 128. Here the selection is exact for every input, and ties are ordered by
// id (smaller first), on a (value, id) key that is unique per element. Two launches:
//   a. brik_topk_prep: each block takes 4096 logits, applies the softcap and the penalty (the recent
//      ids of its range are marked in an LDS bitmap), writes them back, and every lane writes the
//      maximum of its 16 consecutive logits ("lane maxima": maximum q covers logits [16q, 16q + 16)).
//      A q4 / q3 LM head staged once per call runs these passes in its own epilogue instead
//      (gemv.hip, brik_gemvh_*), with the same maxima layout.
//   b. brik_topk_select, one block: folds the lane maxima into 256 maxima of disjoint element sets and
//      takes the k-th largest of those as a bound (k distinct elements reach it, so it is at most the
//      vector's k-th largest; for logits only a few more elements than k pass it). An element at or
//      above the bound lies in a lane whose maximum reaches it, so only those lanes (a few dozen) are
//      read back; each of their elements at or above the bound counts the candidates above it (its
//      rank) and the first k write themselves (a bitonic sort in LDS takes over past 1024 candidates). If the lane or candidate lists overflow (very many equal values at the top), it instead
//      selects the k largest keys by k scans of the whole vector, which is slow but exact.
// No block waits for another inside a launch, so no device-wide fence or counter is needed.
// NaN logits rank below every number (the reference's comparisons never select them either).
#include "common.h"

namespace {

constexpr int TOPK_MAX = 64;
constexpr int TOPK_CAP = 8192;      // candidate list capacity (keys)
constexpr int TOPK_BLOCK = 4096;    // logits per block: 4 waves x 64 lanes x 16

// The order key of common.h (NaN -> 0).
__device__ __forceinline__ uint32_t okey(float v) { return order_key(v); }

__device__ __forceinline__ float okey_inv(uint32_t k)
{
    const uint32_t b = (k & 0x80000000u) ? (k & 0x7fffffffu) : ~k;
    return __builtin_bit_cast(float, b);
}

// (value, id) key: larger value first, then smaller id.
__device__ __forceinline__ uint64_t vkey(uint32_t ok, uint32_t id) { return ((uint64_t)ok << 32) | (0xffffffffu - id); }

// Bitonic sort of s[0, P) (LDS) descending, P a power of two; all NT threads of the block call it.
template <int NT, class K>
__device__ __forceinline__ void bitonic_desc(K* s, int P)
{
    const int tid = threadIdx.x;
    for (int size = 2; size <= P; size <<= 1) {
        for (int stride = size >> 1; stride > 0; stride >>= 1) {
            for (int i = tid; i < P / 2; i += NT) {
                const int a = 2 * i - (i & (stride - 1)), b = a + stride;
                const K x = s[a], y = s[b];
                if ((x < y) == ((a & size) == 0)) {
                    s[a] = y;
                    s[b] = x;
                }
            }
            __syncthreads();
        }
    }
}

}  // namespace

// Block b: logits [4096 b, 4096 b + 4096); thread t: the 16 consecutive logits 4096 b + 16 t + j and
// lane maximum q = 256 b + t.
extern "C" __global__ __launch_bounds__(256) void brik_topk_prep(float* __restrict__ logits, int n, float cap,
                                                                 const int32_t* __restrict__ recent, int n_recent,
                                                                 float penalty, int pen,
                                                                 uint32_t* __restrict__ maxima)
{
    __shared__ uint32_t marks[TOPK_BLOCK / 32];
    const int tid = threadIdx.x;
    const long base = (long)blockIdx.x * TOPK_BLOCK;
    if (pen) {
        for (int i = tid; i < TOPK_BLOCK / 32; i += 256) marks[i] = 0u;
        __syncthreads();
        // ids outside [0, n) are skipped, as sampleNextToken does (src/lib/webgpu/sampling.ts:86)
        for (int r = tid; r < n_recent; r += 256) {
            const long id = recent[r];
            if (id >= base && id < base + TOPK_BLOCK && id < n) {
                const int o = (int)(id - base);
                atomicOr(&marks[o >> 5], 1u << (o & 31));
            }
        }
        __syncthreads();
    }
    // all 16 loads of a thread first (one memory round trip; four at a time took four): four 16-byte
    // buffer loads of a whole chunk (the logits need only 4-byte alignment), else one at a time
    float raw[16];
    const long c0 = base + 16 * tid;
    if (c0 + 16 <= n) {
        const brsrc_t r = make_rsrc(logits, (uint32_t)n * 4u);
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const u32x4_t v = __builtin_amdgcn_raw_buffer_load_b128(r, (uint32_t)(c0 + 4 * u) * 4u, 0, 0);
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const uint32_t w = v[e];      // a scalar first: bit_cast of v[e] itself read element 0
                raw[4 * u + e] = __builtin_bit_cast(float, w);
            }
        }
    } else {
#pragma unroll
        for (int j = 0; j < 16; ++j) raw[j] = c0 + j < n ? logits[c0 + j] : 0.f;
    }
    uint32_t m = 0u;
#pragma unroll
    for (int j = 0; j < 16; ++j) {
        const int o = 16 * tid + j;
        const long i = base + o;
        if (i < n) {
            float v = raw[j];
            const bool p = pen && ((marks[o >> 5] >> (o & 31)) & 1u);
            if (cap > 0.f) v = cap * tanhf(v / cap);
            if (p) v = v > 0.f ? v / penalty : v * penalty;
            if (cap > 0.f || p) logits[i] = v;
            m = max(m, okey(v));
        }
    }
    maxima[(long)blockIdx.x * 256 + tid] = m;
}

constexpr int TOPK_LANES = 2048;    // lanes read back by the select block, at most
constexpr int TOPK_STAGE = 16384;   // lane maxima staged in LDS (vectors of up to 262144 logits)

// One block of 1024 threads; m = the number of lane maxima (256 per prep block, or one per 16 logits
// from a fused LM head), maximum q covering logits [16 q, 16 q + 16).
extern "C" __global__ __launch_bounds__(1024) void brik_topk_select(const float* __restrict__ logits, int n, int k,
                                                                    const uint32_t* __restrict__ maxima, int m,
                                                                    int32_t* __restrict__ out_ids,
                                                                    float* __restrict__ out_vals)
{
    __shared__ uint64_t cand[TOPK_CAP];
    __shared__ uint32_t stage[TOPK_STAGE];
    __shared__ uint32_t folded[256];
    __shared__ uint32_t lanes[TOPK_LANES];
    __shared__ uint32_t counts[3];        // lanes, candidates, bound
    __shared__ uint64_t red[16];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    if (tid < 3) counts[tid] = 0u;
    // the lane maxima, into LDS when they fit (16 loads of a thread in flight at a time)
    const bool staged = m <= TOPK_STAGE;
    if (staged) {
        for (int i0 = 0; i0 < m; i0 += 1024 * 16) {
            uint32_t t[16];
#pragma unroll
            for (int u = 0; u < 16; ++u) {
                const int i = i0 + 1024 * u + tid;
                t[u] = i < m ? maxima[i] : 0u;
            }
#pragma unroll
            for (int u = 0; u < 16; ++u) {
                const int i = i0 + 1024 * u + tid;
                if (i < m) stage[i] = t[u];
            }
        }
    }
    const uint32_t* mx = staged ? stage : maxima;
    // 1. the bound: thread t folds maxima t, t + 1024, ...; groups of 4 threads fold on to 256 values
    uint32_t f = 0u;
    for (int i = tid; i < m; i += 1024) f = max(f, mx[i]);
    f = max(f, (uint32_t)__shfl_xor((int)f, 1));
    f = max(f, (uint32_t)__shfl_xor((int)f, 2));
    if ((tid & 3) == 0) folded[tid >> 2] = f;
    __syncthreads();
    // the k-th largest of the 256 folded values: the largest T with at least k values >= T, built bit by
    // bit from the top (the count is monotone in T), by wave 0 with ballots
    if (wave == 0) {
        uint32_t v[4], T = 0u;
#pragma unroll
        for (int u = 0; u < 4; ++u) v[u] = folded[lane + 64 * u];
        for (int bit = 31; bit >= 0; --bit) {
            const uint32_t t = T | (1u << bit);
            int c = 0;
#pragma unroll
            for (int u = 0; u < 4; ++u) c += __builtin_popcountll(__ballot(v[u] >= t));
            if (c >= k) T = t;
        }
        if (lane == 0) counts[2] = T;
    }
    __syncthreads();
    const uint32_t bound = counts[2];
    // 2. the lanes whose maxima reach it
    for (int i = tid; i < m; i += 1024) {
        if (mx[i] >= bound) {
            const uint32_t at = atomicAdd(&counts[0], 1u);
            if (at < (uint32_t)TOPK_LANES) lanes[at] = (uint32_t)i;
        }
    }
    __syncthreads();
    const uint32_t nl = counts[0];
    bool overflow = nl > (uint32_t)TOPK_LANES;
    // 3. their elements at or above the bound
    if (!overflow) {
        for (uint32_t e = tid; e < nl * 16u; e += 1024) {
            const uint32_t q = lanes[e >> 4], j = e & 15u;
            const long i = 16L * q + j;
            if (i < n) {
                const uint32_t key = okey(logits[i]);
                if (key >= bound) {
                    const uint32_t at = atomicAdd(&counts[1], 1u);
                    if (at < (uint32_t)TOPK_CAP) cand[at] = vkey(key, (uint32_t)i);
                }
            }
        }
        __syncthreads();
        overflow = counts[1] > (uint32_t)TOPK_CAP;
    }
    if (!overflow) {
        const uint32_t cnt = counts[1];
        if (cnt <= 1024u) {
            // rank of each candidate among the others (keys are unique); the first k write themselves
            if ((uint32_t)tid < cnt) {
                const uint64_t me = cand[tid];
                uint32_t rank = 0u;
                for (uint32_t j = 0; j < cnt; ++j) rank += cand[j] > me;
                if (rank < (uint32_t)k) {
                    out_ids[rank] = (int32_t)(0xffffffffu - (uint32_t)me);
                    out_vals[rank] = okey_inv((uint32_t)(me >> 32));
                }
            }
            return;
        }
        int P = 2048;
        while ((uint32_t)P < cnt) P <<= 1;
        for (int i = tid; i < P; i += 1024)
            if ((uint32_t)i >= cnt) cand[i] = 0ull;
        __syncthreads();
        bitonic_desc<1024>(cand, P);
        if (tid < k) {
            const uint64_t v = cand[tid];
            out_ids[tid] = (int32_t)(0xffffffffu - (uint32_t)v);
            out_vals[tid] = okey_inv((uint32_t)(v >> 32));
        }
        return;
    }
    // overflow: k scans, each taking the largest key below the previous one
    uint64_t prev = ~0ull;
    for (int r = 0; r < k; ++r) {
        uint64_t best = 0ull;
        for (long i = tid; i < n; i += 1024) {
            const uint64_t v = vkey(okey(logits[i]), (uint32_t)i);
            if (v < prev && v > best) best = v;
        }
        for (int o = 32; o > 0; o >>= 1) {
            const uint64_t t = ((uint64_t)(uint32_t)__shfl_xor((int)(best >> 32), o) << 32) |
                               (uint32_t)__shfl_xor((int)(uint32_t)best, o);
            best = t > best ? t : best;
        }
        if (lane == 0) red[wave] = best;
        __syncthreads();
        uint64_t b = red[0];
        for (int w = 1; w < 16; ++w) b = red[w] > b ? red[w] : b;
        if (tid == 0) {
            out_ids[r] = (int32_t)(0xffffffffu - (uint32_t)b);
            out_vals[r] = okey_inv((uint32_t)(b >> 32));
        }
        prev = b;
        __syncthreads();
    }
}
