// screen_kernels.hip -- fp16 screen ahead of an fp32 collect pass.
//
// A collect pass over fp32 rows collects, for every query q of a 128-query
// work item, the keys of the item's pool at or below a threshold T_q (the
// running M-th distance of a seeded pass), then selects the M smallest
// (knn_f32_collect_kernel).  The screen computes every (q, p) pair of the
// item on the fp16 matrix cores (v_mfma_f32_32x32x16_f16: rows scaled by one
// power of two 2^k for the whole matrix, rounded to fp16, fp32 sums) and
// keeps the pool rows p whose fp16 key minus a rigorous bound e(q, p) on its
// gap to the fp32 path's key is at most T_q for some query of the item: every
// row whose fp32 key is at or below T_q is kept.  The union of kept rows, in
// pool order, becomes the item's pool for the fp32 collect pass, which
// therefore collects exactly the keys the full pool would give it (its keys
// are per pair and ordered by (key, id), so neither the rows it no longer
// visits nor the visiting order change a list).  An unseeded pass first
// bounds each query's M-th smallest fp32 key from above with fp16 keys plus e
// over the item's first tiles (the window) and is then screened and collected
// against that bound: the lists are the unscreened pass's bit for bit.
//
// The scale: k = 15 - E with max_x |x| < 2^E, so every scaled element is
// below 2^15 (fp16's largest finite value is 65504); products of fp16 values
// are exact in fp32 and scaled dot products stay below 2^38.  Keys and norms
// scale by 4^k and 2^k exactly (powers of two) except where they underflow.
//
// The bound, in scaled units.  S = sum_i |q_i p_i| <= |q| |p|
// (Cauchy-Schwarz).  Rounding to fp16 moves an element by at most 2^-11 of
// itself plus 2^-14 (subnormals, flushed or not), so
//   |sum q~_i p~_i - sum q_i p_i| <= (2^-10 + 2^-22) S + 2^-14 (1 + 2^-11) (|q|_1 + |p|_1) + D 2^-28
// with |x|_1 <= sqrt(D) |x| < 16 |x| (D <= 160): below
// (2^-10 + 2^-22) S + 2^-10 (|q| + |p|) + 2^-20.  Either path's fp32 sums
// over D terms (in any order, each add within 2^-23 of its result, truncating
// adds included) add at most D 2^-23 (1 + 2^-10) S < 2^-15.6 S each, so the
// dot products differ by less than c S + 2^-10 (|q| + |p|) + 2^-20 with
// c = 2^-10 + 2^-12 (which leaves 2^-12.6 S for matrix-core sums coarser than
// that).  The fp32 key's own roundings (|q|^2 + |p|^2, then one fma; results
// of at most 2 (|q|^2 + |p|^2)) and the roundings of the tests below add less
// than R (|q|^2 + |p|^2), R = 2^-19 (L2).  With d the fp16 dot, A = 2^-20:
//   L2 (key |q|^2 + |p|^2 - 2 q.p):  e = 2 c |q||p| + 2^-9 (|q| + |p|) + R (|q|^2 + |p|^2) + A
//   IP (key -q.p):                    e = (c + R) |q||p| + 2^-10 (|q| + |p|) + A
// |x| is sqrt of the fp32 |x|^2 both paths use (within 2^-23 relative of the
// true norm, inside the spare of c).  "fp16 key - e <= T" is evaluated as
//   L2: fma(2, d, fma(cq, |p|, -(1 - R) |p|^2)) >= (1 - R) |q|^2 - T - A - 2^-9 |q|,   cq = 2 c |q| + 2^-9
//   IP: fma(cq, |p|, d)                         >= -T - A - 2^-10 |q|,                 cq = (c + R) |q| + 2^-10
// (two and one vector instructions per pair before the compare), and the
// window's upper bound "fp16 key + e" as
//   L2: fma(-2, d, fma(cq, |p|, (1 + R) |p|^2 + (1 + R) |q|^2 + A + 2^-9 |q|))
//   IP: fma(cq, |p|, A + 2^-10 |q| - d).
// T = +inf keeps every row; a matrix whose largest norm is not finite or
// needs |k| > 60 is not screened (every row kept, every window bound +inf).
#include "knn_device.hpp"

#include <algorithm>

namespace gtann {

typedef _Float16 halfx8 __attribute__((ext_vector_type(8)));
typedef float floatx16 __attribute__((ext_vector_type(16)));

constexpr int kScreenMaxPool = 32768;   // pool rows an item's LDS bitmap covers
constexpr float kScreenC = 0x1p-10f + 0x1p-12f;
constexpr float kScreenR = 0x1p-19f;
constexpr float kScreenA = 0x1p-20f;
constexpr float kScreenD = 0x1p-10f;   // the subnormal term's factor (per metric: x2 for L2)
constexpr float kScreenAOut = 0x1p-60f;   // added to a window bound returned unscaled

// max over rows of |x|^2 (non-negative floats order as their bit patterns)
__global__ void __launch_bounds__(256) screen_norm_max_kernel(const float* __restrict__ nrm, int64_t N,
                                                             unsigned int* __restrict__ out)
{
    unsigned int m = 0u;
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; i < N;
         i += static_cast<int64_t>(gridDim.x) * 256) {
        const float v = nrm[i];
        m = max(m, v >= 0.f ? __float_as_uint(v) : 0x7F800000u);   // NaN: not finite
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) m = max(m, static_cast<unsigned int>(__shfl_xor(static_cast<int>(m), o)));
    if ((threadIdx.x & 63) == 0) atomicMax(out, m);
}

// The scale exponent k from the largest |x|^2 (scale[0] = k, scale[1] = 1
// when the matrix cannot be screened).
__device__ __forceinline__ void screen_scale(const unsigned int* sq, int& k, bool& off)
{
    const float n2 = __uint_as_float(*sq);
    off = !(n2 < INFINITY);
    int E = 0;
    if (!off && n2 > 0.f) {
        frexpf(sqrtf(n2) * 1.0000002f, &E);   // max |x| < 2^E (the factor: sqrt's rounding)
    }
    k = 15 - E;
    if (k < -60 || k > 60) off = true;
    if (off) k = 0;
}

// fp32 rows (stride Dp) -> 2^k-scaled fp16 rows (stride Dp), round to nearest even
__global__ void __launch_bounds__(256) screen_f16_kernel(const float4* __restrict__ X, int64_t n4,
                                                        const unsigned int* __restrict__ sq, uint2* __restrict__ Xh)
{
    int k;
    bool off;
    screen_scale(sq, k, off);
    const float sc = ldexpf(1.f, k);
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; i < n4;
         i += static_cast<int64_t>(gridDim.x) * 256) {
        const float4 v = X[i];
        const _Float16 h0 = static_cast<_Float16>(off ? 0.f : v.x * sc);
        const _Float16 h1 = static_cast<_Float16>(off ? 0.f : v.y * sc);
        const _Float16 h2 = static_cast<_Float16>(off ? 0.f : v.z * sc);
        const _Float16 h3 = static_cast<_Float16>(off ? 0.f : v.w * sc);
        const uint32_t b0 = __builtin_bit_cast(uint16_t, h0), b1 = __builtin_bit_cast(uint16_t, h1);
        const uint32_t b2 = __builtin_bit_cast(uint16_t, h2), b3 = __builtin_bit_cast(uint16_t, h3);
        Xh[i] = make_uint2(b0 | (b1 << 16), b2 | (b3 << 16));
    }
}

// One block per work item (4 waves of 32 queries; lanes j and j + 32 hold
// query j's dims 16 s + 8 h + [0, 8) of step s, h = lane / 32).  Pool tiles
// of 32 rows are staged through LDS, double buffered (the next tile's loads
// in flight during a tile's MFMAs).  In the admission scan the queries are
// the MFMA's rows: a tile's accumulator element 4 g + e of lane (j, h) is pool
// row j against query 8 g + 4 h + e; the 16 compares' lane masks OR into the
// tile's admitted rows (bit j from lanes j and j + 32), which each wave ORs
// into word t of the item's LDS bitmap; the set bits, in pool order, become
// the item's union at union_rows[ubase[item] ...).
template <int DP, int METRIC, bool WINDOW>
__global__ void __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(WINDOW || DP > 128 ? 2 : 4))) knn_screen_kernel(const WorkItem* __restrict__ items,
                                                         const int32_t* __restrict__ pairs,
                                                         const int64_t* __restrict__ ubase,
                                                         const int32_t* __restrict__ q_rows,
                                                         const int32_t* __restrict__ p_rows,
                                                         const uint16_t* __restrict__ Xh, const float* __restrict__ nrm,
                                                         const unsigned int* __restrict__ sq,
                                                         const float* __restrict__ seed_d, int seed_ld, int M,
                                                         int wtiles, float* __restrict__ tq,
                                                         int32_t* __restrict__ union_rows,
                                                         WorkItem* __restrict__ items_out,
                                                         unsigned long long* __restrict__ pairs_done)
{
    constexpr int KS = DP / 16;          // MFMA steps per tile
    constexpr int RS = DP + 8;           // LDS row stride (fp16 elements): rows on distinct bank groups
    constexpr int U4_ROW = DP / 8;       // 16-byte pieces per row
    constexpr int U4_TILE = kPoolTile * U4_ROW;
    constexpr int NT = WINDOW ? 256 : 512;           // threads: one item, or a pair sharing the pool
    constexpr int U4_THREAD = (U4_TILE + NT - 1) / NT;
    constexpr int WPT = kScreenMaxPool / 32 / 256;   // bitmap words per thread in the compaction
    static_assert(DP % 16 == 0 && kPoolTile == 32, "fp16 steps of 16 dims, one bitmap word per tile");
    __shared__ __align__(16) uint16_t tile[2][kPoolTile][RS];
    __shared__ __align__(16) float tpr[2][kPoolTile];   // |p|
    __shared__ __align__(16) float tpm[2][kPoolTile];   // -(1 - R) |p|^2
    __shared__ __align__(16) float tpu[2][kPoolTile];   // (1 + R) |p|^2
    __shared__ __align__(16) int32_t trow[2][kPoolTile];   // row id, -1 past the pool's end
    __shared__ uint32_t bits[2][kScreenMaxPool / 32];   // per item of the pair
    __shared__ uint32_t wsum[2][kWaves];
    __shared__ uint32_t urot[2];

    // the items (window) or pairs (admission) are laid out XCD by XCD (an
    // eighth each, a bucket's together): block b runs entry
    // (b mod 8) (n / 8) + b / 8, so the blocks one XCD runs share their pools
    // in its L2.  An admission block runs two items of one pool (waves 0-3
    // the first, 4-7 the second), each staged pool tile serving both.
    const int per = static_cast<int>(gridDim.x) / 8;
    const int entry = static_cast<int>(blockIdx.x % 8) * per + static_cast<int>(blockIdx.x / 8);
    const int tid = threadIdx.x;
    const int w = tid >> 6, lane = tid & 63, j = lane & 31, h = lane >> 5;
    const int half = WINDOW ? 0 : w >> 2, wq = w & 3;
    int item_idx, pool_idx;
    if constexpr (WINDOW) {
        item_idx = pool_idx = entry;
    } else {
        pool_idx = pairs[2 * entry];
        item_idx = pairs[2 * entry + half];
        if (pool_idx < 0) return;   // padding
    }
    const WorkItem pool = items[pool_idx];
    const WorkItem it = items[item_idx >= 0 ? item_idx : pool_idx];
    const int nq = item_idx >= 0 ? it.q_count : 0;   // 0: the pair's missing second item
    if (WINDOW && nq <= 0) return;   // padding
    const int pc = pool.p_count;
    const int ntiles = (pc + kPoolTile - 1) / kPoolTile;
    if (!WINDOW)
        for (int i = tid; i < ntiles; i += NT) bits[0][i] = bits[1][i] = 0u;

    const int qlocal = wq * kQueriesPerWave + j;
    const bool qvalid = qlocal < nq;
    const int64_t qi = it.q_begin + qlocal;
    const int32_t qrow = qvalid ? (q_rows ? q_rows[qi] : static_cast<int32_t>(qi)) : 0;
    const int64_t orow = it.out_base >= 0 ? it.out_base + qlocal : static_cast<int64_t>(qrow);
    int k;
    bool unscreened;   // the matrix's scale is out of range: every row kept
    screen_scale(sq, k, unscreened);
    const float s1 = ldexpf(1.f, k), s2 = ldexpf(1.f, 2 * k);   // exact powers of two
    const float qn = nrm[qrow] * s2;
    const float qr = sqrtf(nrm[qrow]) * s1;
    constexpr float kD = METRIC == 0 ? 2.f * kScreenD : kScreenD;
    const float cq = METRIC == 0 ? fmaf(2.f * kScreenC, qr, kD) : fmaf(kScreenC + kScreenR, qr, kD);
    halfx8 qf[KS];
    {
        const uint4* src = reinterpret_cast<const uint4*>(Xh + static_cast<int64_t>(qrow) * DP + 8 * h);
#pragma unroll
        for (int s = 0; s < KS; ++s) qf[s] = __builtin_bit_cast(halfx8, src[2 * s]);
    }

    // pool tile t: positions rot + 32 t + r (mod pc) for 32 t + r < pc,
    // flowing through row ids (fetched a tile ahead of the row loads, so a
    // row load never waits on an id load) -> rows and norms in registers
    // (two register sets: loaded two tiles ahead of their use) -> LDS (two
    // buffers).  fetch_ids(t) loads tile t's ids; load_into(set) issues the
    // loads of the tile fetch_ids last named; store_from(set, buf) puts a set
    // into LDS.
    int32_t idq[U4_THREAD];   // ids of the next tile's 16-byte pieces (-1: none)
    int32_t ridq = -1;        // threads < 32: the id of the next tile's row tid
    struct Set {
        uint4 v[U4_THREAD];
        int32_t rid;
        float pn;
    };
    Set set0, set1;
    set0.rid = set1.rid = -1;
    set0.pn = set1.pn = 0.f;
    auto pos_row = [&](int t, int r, int rot) __attribute__((always_inline)) -> int32_t {
        int p = t * kPoolTile + r;
        if (p >= pc) return -1;
        p += rot;
        if (p >= pc) p -= pc;
        return p_rows[pool.p_begin + p];
    };
    auto fetch_ids = [&](int t, int rot) __attribute__((always_inline)) {
#pragma unroll
        for (int u = 0; u < U4_THREAD; ++u) {
            const int e = tid + NT * u;
            idq[u] = e < U4_TILE ? pos_row(t, e / U4_ROW, rot) : -1;
        }
        if (tid < kPoolTile) ridq = pos_row(t, tid, rot);
    };
    auto load_into = [&](Set& S) __attribute__((always_inline)) {
#pragma unroll
        for (int u = 0; u < U4_THREAD; ++u) {
            const int e = tid + NT * u;
            S.v[u] = idq[u] >= 0 ? reinterpret_cast<const uint4*>(Xh + static_cast<int64_t>(idq[u]) * DP)[e % U4_ROW]
                                 : make_uint4(0u, 0u, 0u, 0u);
        }
        if (tid < kPoolTile) {
            S.rid = ridq;
            S.pn = ridq >= 0 ? nrm[ridq] : 0.f;
        }
    };
    auto store_from = [&](const Set& S, int buf) __attribute__((always_inline)) {
#pragma unroll
        for (int u = 0; u < U4_THREAD; ++u) {
            const int e = tid + NT * u;
            if (e < U4_TILE) *reinterpret_cast<uint4*>(&tile[buf][e / U4_ROW][8 * (e % U4_ROW)]) = S.v[u];
        }
        if (tid < kPoolTile) {
            tpr[buf][tid] = sqrtf(S.pn) * s1;
            tpm[buf][tid] = -(1.f - kScreenR) * (S.pn * s2);
            tpu[buf][tid] = (1.f + kScreenR) * (S.pn * s2);
            trow[buf][tid] = S.rid;
        }
    };
    // runs body(t, buf) over tiles 0 .. n - 1 (tile t in LDS buffer t & 1),
    // one barrier per tile
    auto pipeline = [&](int n, int rot, auto&& body) __attribute__((always_inline)) {
        if (n > 0) {
            fetch_ids(0, rot);
            load_into(set0);
        }
        if (n > 1) {
            fetch_ids(1, rot);
            load_into(set1);
        }
        if (n > 2) fetch_ids(2, rot);
        if (n > 0) store_from(set0, 0);
        __syncthreads();
        for (int t = 0; t < n; t += 2) {
            if (t + 2 < n) {
                load_into(set0);
                if (t + 3 < n) fetch_ids(t + 3, rot);
            }
            body(t, 0);
            if (t + 1 < n) store_from(set1, 1);
            __syncthreads();
            if (t + 1 < n) {
                if (t + 3 < n) {
                    load_into(set1);
                    if (t + 4 < n) fetch_ids(t + 4, rot);
                }
                body(t + 1, 1);
                if (t + 2 < n) store_from(set0, 0);
                __syncthreads();
            }
        }
    };

    // WINDOW: an upper bound on the M-th smallest fp32 key of the pool from
    // its first wtiles tiles (from the item's rotation), to tq: each lane
    // keeps the 32 smallest bounds ub = fp16 key + e >= fp32 key of the rows
    // it holds (a sorting network on registers), and the larger of the pair's
    // ceil(M/2)-th smallest bounds ceil(M/2) rows of each lane from above: M
    // distinct rows, the query itself excluded (+inf if the window has fewer).
    // Else the admission scan against the query's threshold seed_d (the
    // running M-th distance, or such a bound; +inf keeps every row).
    if constexpr (WINDOW) {
        const float qk = METRIC == 0 ? fmaf(kD, qr, (1.f + kScreenR) * qn + kScreenA) : fmaf(kD, qr, kScreenA);
        float L[32];
#pragma unroll
        for (int i = 0; i < 32; ++i) L[i] = INFINITY;
        const int nwt = min(wtiles, ntiles);
        pipeline(nwt, it.p_rot, [&](int t, int buf) __attribute__((always_inline)) {
            floatx16 acc;
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[r] = 0.f;
            // pool rows as A, queries as B: element 4 g + e of lane (j, h)
            // is pool row 8 g + 4 h + e against query j
            const uint16_t* arow = &tile[buf][j][8 * h];
#pragma unroll
            for (int s = 0; s < KS; ++s) {
                const halfx8 av = __builtin_bit_cast(halfx8, *reinterpret_cast<const uint4*>(arow + 16 * s));
                acc = __builtin_amdgcn_mfma_f32_32x32x16_f16(av, qf[s], acc, 0, 0, 0);
            }
            float ub[16];
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                const float4 r4 = *reinterpret_cast<const float4*>(&tpr[buf][8 * g + 4 * h]);
                const float4 u4 = *reinterpret_cast<const float4*>(&tpu[buf][8 * g + 4 * h]);
                const int4 i4 = *reinterpret_cast<const int4*>(&trow[buf][8 * g + 4 * h]);
                const float pr[4] = {r4.x, r4.y, r4.z, r4.w}, pu[4] = {u4.x, u4.y, u4.z, u4.w};
                const int32_t id[4] = {i4.x, i4.y, i4.z, i4.w};
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const float d = acc[4 * g + e];
                    const float v = METRIC == 0 ? fmaf(-2.f, d, fmaf(cq, pr[e], pu[e] + qk)) : fmaf(cq, pr[e], qk - d);
                    ub[4 * g + e] = (id[e] < 0 || id[e] == qrow || !(v < INFINITY)) ? INFINITY : v;   // NaN: no bound
                }
            }
            oddeven_sort(ub);
#pragma unroll
            for (int k = 0; k < 16; ++k) L[16 + k] = fminf(L[16 + k], ub[15 - k]);
            bitonic_merge(L);
        });
        const int m = (M + 1) / 2 - 1;
        float v = L[0];
#pragma unroll
        for (int i = 1; i < 32; ++i) v = i == m ? L[i] : v;
        v = fmaxf(v, __shfl_xor(v, 32));
        // unscaled (exact but for underflow, which the added 2^-60 covers)
        if (qvalid && h == 0) tq[orow] = unscreened ? INFINITY : fmaf(v, ldexpf(1.f, -2 * k), kScreenAOut);
        return;
    }
    const float T = qvalid ? (unscreened ? INFINITY : seed_d[orow * seed_ld + seed_ld - 1] * s2) : 0.f;
    // an invalid query admits nothing (y >= +inf fails for every finite y)
    const float qa = !qvalid ? INFINITY
                     : METRIC == 0 ? fmaf(-kD, qr, qn * (1.f - kScreenR) - T - kScreenA)
                                   : fmaf(-kD, qr, -T - kScreenA);
    // the constants of the queries this lane's accumulator elements hold
    // in the admission scan (element 4 g + e: query 8 g + 4 h + e)
    float qa_r[16], cq_r[16];
#pragma unroll
    for (int r = 0; r < 16; ++r) {
        const int src = 8 * (r >> 2) + 4 * h + (r & 3);
        qa_r[r] = __shfl(qa, src);
        cq_r[r] = __shfl(cq, src);
    }

    pipeline(ntiles, 0, [&](int t, int buf) __attribute__((always_inline)) {
        floatx16 acc;
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[r] = 0.f;
        // queries as A (rows), pool rows as B (columns): lane (j, h) ends
        // with pool row j against queries 8 g + 4 h + e
        const uint16_t* brow = &tile[buf][j][8 * h];
#pragma unroll
        for (int s = 0; s < KS; ++s) {
            const halfx8 bv = __builtin_bit_cast(halfx8, *reinterpret_cast<const uint4*>(brow + 16 * s));
            acc = __builtin_amdgcn_mfma_f32_32x32x16_f16(qf[s], bv, acc, 0, 0, 0);
        }
        const float pr = tpr[buf][j], pm = tpm[buf][j];
        uint64_t m = 0u;   // lanes whose pool row some query admits
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const float y = METRIC == 0 ? fmaf(2.f, acc[r], fmaf(cq_r[r], pr, pm)) : fmaf(cq_r[r], pr, acc[r]);
            m |= __ballot(y >= qa_r[r]);
        }
        uint32_t tm = static_cast<uint32_t>(m) | static_cast<uint32_t>(m >> 32);   // bit j: pool row j
        const int left = pc - t * kPoolTile;
        if (left < kPoolTile) tm &= (1u << left) - 1u;
        if (lane == 0 && tm) atomicOr(&bits[half][t], tm);
    });
    // the set bits of each item's bitmap, in order, as row ids (threads
    // 256 half .. 256 half + 255 for item half)
    const int th = tid & 255;
    uint32_t cnt = 0u;
#pragma unroll
    for (int u = 0; u < WPT; ++u) {
        const int wi = th * WPT + u;
        cnt += wi < ntiles ? static_cast<uint32_t>(__popc(bits[half][wi])) : 0u;
    }
    uint32_t inc = cnt;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const uint32_t x = __shfl_up(inc, o);
        if (lane >= o) inc += x;
    }
    if (lane == 63) wsum[half][wq] = inc;
    __syncthreads();
    uint32_t off = inc - cnt;
    for (int q = 0; q < wq; ++q) off += wsum[half][q];
    // the union's rotation: its first row at or after the item's rotation
    // (an unseeded fp32 pass takes its threshold window from there)
    const int wr = it.p_rot >> 5;
    if (item_idx >= 0 && pc > 0 && th == wr / WPT) {
        uint32_t r = off;
        for (int wi = th * WPT; wi < wr; ++wi) r += static_cast<uint32_t>(__popc(bits[half][wi]));
        urot[half] = r + static_cast<uint32_t>(__popc(bits[half][wr] & ((1u << (it.p_rot & 31)) - 1u)));
    }
    __syncthreads();
    if (item_idx < 0) return;
    const int64_t base = ubase[item_idx];
#pragma unroll
    for (int u = 0; u < WPT; ++u) {
        const int wi = th * WPT + u;
        uint32_t b = wi < ntiles ? bits[half][wi] : 0u;
        while (b) {
            const int k = __ffs(b) - 1;
            b &= b - 1u;
            union_rows[base + off++] = p_rows[pool.p_begin + wi * 32 + k];
        }
    }
    if (th == 0) {
        WorkItem o = it;
        o.p_begin = base;
        o.p_count = static_cast<int32_t>(wsum[half][0] + wsum[half][1] + wsum[half][2] + wsum[half][3]);
        o.p_rot = pc > 0 && static_cast<int32_t>(urot[half]) < o.p_count ? static_cast<int32_t>(urot[half]) : 0;
        items_out[item_idx] = o;
        if (pairs_done)
            atomicAdd(pairs_done, static_cast<unsigned long long>(o.p_count) * static_cast<unsigned>(o.q_count));
    }
}

bool screen_supported(int Dp, int64_t max_pool)
{
    return (Dp == 32 || Dp == 64 || Dp == 96 || Dp == 128 || Dp == 160) && max_pool <= kScreenMaxPool;
}

// Xh: the 2^k-scaled fp16 copy of X (N rows, stride Dp); sq: one unsigned
// int of device memory for the scale (written here)
void launch_screen_prepare(const float* X, const float* nrm, int64_t N, int Dp, unsigned int* sq, uint16_t* Xh,
                           hipStream_t s)
{
    GT_REQUIRE(Dp % 4 == 0, "screen: rows of whole float4s");
    if (N <= 0) return;
    GT_HIP(hipMemsetAsync(sq, 0, sizeof(unsigned int), s));
    const unsigned g1 = static_cast<unsigned>(std::min<int64_t>(ceil_div(N, int64_t(256)), 1024));
    hipLaunchKernelGGL(screen_norm_max_kernel, dim3(g1), dim3(256), 0, s, nrm, N, sq);
    GT_HIP(hipGetLastError());
    const int64_t n4 = N * Dp / 4;
    const unsigned grid = static_cast<unsigned>(std::min<int64_t>(ceil_div(n4, int64_t(256)), 8192));
    hipLaunchKernelGGL(screen_f16_kernel, dim3(grid), dim3(256), 0, s, reinterpret_cast<const float4*>(X), n4, sq,
                       reinterpret_cast<uint2*>(Xh));
    GT_HIP(hipGetLastError());
}

// items: n_items work items of a pass (every pool at most kScreenMaxPool
// rows); pairs: n_pairs entries (first item, second item or -1; -1, -1 for
// padding) pairing every item that has queries with at most one other item
// of the same pool, laid out like the items; ubase[i]: item i's first slot
// of union_rows, which holds at least
// its pool count from there; items_out: the items with their unions as pools
// (rotated to the union's first row at or after the item's rotation).  Xh:
// the scaled fp16 rows (stride Dp) of the matrix the q_rows and p_rows
// index, sq its scale (launch_screen_prepare), nrm its fp32 |x|^2.  A seeded
// pass (seed_d: running tables of seed_ld keys per output row) screens
// against each row's last key; an unseeded one (M keys wanted, 4 < M <= 64)
// against a bound from the first wtiles tiles of each item's rotated pool,
// written to tq (one per output row: the pool's M-th smallest fp32 key is at
// or below it).  pairs_done (optional) += the (query, union row) pairs left
// to the fp32 pass.
void launch_screen(const WorkItem* items, int n_items, const int32_t* pairs, int n_pairs, const int64_t* ubase,
                   const int32_t* q_rows,
                   const int32_t* p_rows, const uint16_t* Xh, const float* nrm, const unsigned int* sq, int Dp,
                   int metric, const float* seed_d, int seed_ld, int M, int wtiles, float* tq, int32_t* union_rows,
                   WorkItem* items_out, unsigned long long* pairs_done, hipStream_t s)
{
    GT_REQUIRE(screen_supported(Dp, 0), "screen: padded dimension not supported");
    GT_REQUIRE(n_items % 8 == 0 && n_pairs % 8 == 0, "screen: work lists must be padded to multiples of 8 (one eighth per XCD)");
    GT_REQUIRE(pairs != nullptr, "screen: item pairs missing");
    // the items without a pair entry (padding) keep their pools
    GT_HIP(hipMemcpyAsync(items_out, items, static_cast<size_t>(n_items) * sizeof(WorkItem), hipMemcpyDeviceToDevice, s));
    GT_REQUIRE(seed_d ? seed_ld > 0 : (tq && M > 4 && M <= 64 && wtiles > 0), "screen: seed or window missing");
    if (n_items <= 0) return;
#define GT_SCR(DPV, MET)                                                                                      \
    do {                                                                                                      \
        if (!seed_d)                                                                                          \
            hipLaunchKernelGGL((knn_screen_kernel<DPV, MET, true>), dim3(n_items), dim3(256), 0, s, items,    \
                               nullptr, ubase, q_rows, p_rows, Xh, nrm, sq, seed_d, seed_ld, M, wtiles, tq,    \
                               union_rows, items_out, pairs_done);                                            \
        const float* sd = seed_d ? seed_d : tq;                                                               \
        const int sl = seed_d ? seed_ld : 1;                                                                  \
        hipLaunchKernelGGL((knn_screen_kernel<DPV, MET, false>), dim3(n_pairs), dim3(512), 0, s, items, pairs, \
                           ubase, q_rows, p_rows, Xh, nrm, sq, sd, sl, M, wtiles, tq, union_rows, items_out,    \
                           pairs_done);                                                                       \
    } while (0)
#define GT_SCR_M(DPV)                     \
    do {                                  \
        if (metric == 0) GT_SCR(DPV, 0);  \
        else GT_SCR(DPV, 1);              \
    } while (0)
    switch (Dp) {
    case 32: GT_SCR_M(32); break;
    case 64: GT_SCR_M(64); break;
    case 96: GT_SCR_M(96); break;
    case 128: GT_SCR_M(128); break;
    default: GT_SCR_M(160); break;
    }
#undef GT_SCR_M
#undef GT_SCR
    GT_HIP(hipGetLastError());
}

}  // namespace gtann
