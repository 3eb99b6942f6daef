// knn_collect.hip -- per-bucket brute-force kNN as collect + select, for
// lists of 5..64 keys on int8 rows (Dp <= 256) and on fp32 rows (Dp <= 160)
// (src/bucket.cu:4101-4265 top-M semantics: self excluded, (-1, +inf)
// padding, ties by id).
//
// knn_i8_collect_kernel scans a tile of 128 queries against a pool slice like
// knn_i8_kernel (int8 MFMA, LDS pool tiles, integer pre-filter) but keeps no
// list: every key at or below the query's threshold is appended to the
// query's candidate slots in HBM.  The threshold is the caller's cap (the
// running M-th distance of a seeded pass) or, in an unseeded pass, a bound
// taken from the first tiles of the scan (the window): each lane keeps the 32
// smallest distances among the pool rows it holds in those tiles (a sorting
// network on registers), and the larger of the pair's ceil(M/2)-th smallest
// bounds the pool's M-th smallest from above (those are M distinct rows).
// The scan then visits the whole slice (the window's tiles last).  A query
// whose slots fill up is compacted by its wave: the M-th smallest of its keys
// is found by a radix descent over the 64 key bits, the keys above it are
// dropped and it becomes the threshold.  The kept set always contains the
// pool's M smallest keys at or below the cap, so the selection that follows
// gives the same list as a scan that merges as it goes.
//
// knn_select_kernel sorts each query's candidates into its top-M list: two
// lanes per query merge 32 keys at a time into a sorted register list
// (pair_merge32).
#include "knn_device.hpp"

#include <climits>
#include <cstdlib>
#include <type_traits>

namespace gtann {

// tiles (of kPoolTile pool rows) of the unseeded threshold pass: the
// caller's KnnArgs::window_tiles (even, at most kWindowMax), else kWindow
constexpr int kWindow = 16;
constexpr int kWindowMax = 32;
__device__ __forceinline__ int window_tiles(const KnnArgs& a)
{
    return a.window_tiles > 0 ? min(a.window_tiles, kWindowMax) & ~1 : kWindow;
}

// Per-wave staging of a tile's candidates: every lane's 16 accumulators
// (16-byte chunks swizzled by lane so that a wave's 128-bit stores spread
// over the banks), one 16-bit code (lane << 4 | element) per accumulator at
// or above its lane's pass floor (plus a spare slot per lane), the wave's
// queries' slot counters and the query state the dense pass reads.
constexpr int kCodeSpare = 64 * 16;   // first of the 64 per-lane spare code slots

struct CollectWave {
    int32_t stash[64 * 16];
    uint16_t code[kCodeSpare + 64];
    int32_t qcnt[kQueriesPerWave];
    float4 qst[kQueriesPerWave];          // |q|^2, threshold, threshold id (bits), self (bits)
    int64_t qrow_out[kQueriesPerWave];    // output row
};

constexpr int kStageTiles = 2;                       // tiles (of kPoolTile pool rows) per pipeline stage
constexpr int kStageRows = kPoolTile * kStageTiles;

template <int DP>
struct CollectSmem {
    int8_t tile[2][kStageRows][DP + 16];   // +16 bytes: rows land on distinct bank groups
    float tnorm[3][kStageRows];
    int32_t trow[3][kStageRows];
    int32_t thalf[3][kStageRows];          // accumulator start: -floor(|p|^2 / 2) (L2), 0 (IP), kHalfPast past the end
    int32_t sid[2][kStageRows];            // the next stage's pool row ids, for every thread's row requests
    CollectWave wv[kWaves];
    // chunk pruning: each wave's chunks needed (bits), the block's, and the
    // schedule of the stages still to scan
    uint32_t wmask[kWaves][kMaxChunkWords];
    uint32_t bmask[kMaxChunkWords];
    uint16_t slist[kMaxChunkWords * 32 + kWindowMax / kStageTiles + 2];
    int32_t nlist;
};
static_assert(kChunkRows == kStageRows, "a pruning chunk is one stage of pool rows");

__device__ __forceinline__ int stash_index(int lane, int r)
{
    return lane * 16 + (((r >> 2) ^ ((lane >> 1) & 3)) << 2) + (r & 3);
}

// Per-lane view of one query (lanes j and j + 32 hold identical copies).
struct CollectState {
    float thr;          // a key passes iff (d, id) <= (thr, thr_id)
    uint32_t thr_id;    // 0xffffffff: every id at distance thr
    int32_t cnt;        // keys in the query's slots
    int32_t self;       // id that must not be kept (the query itself), -2 if none
    int64_t orow;       // output row
};

__device__ __forceinline__ bool key_passes(float d, int32_t id, const CollectState& st)
{
    return d < st.thr || (d == st.thr && static_cast<uint32_t>(id) <= st.thr_id);
}

// Keeps the M smallest of query q's cnt (> M) keys in its slots and makes the
// M-th its threshold.  Called by all 64 lanes; q is uniform.
__device__ __forceinline__ void collect_compact(const KnnArgs& a, int lane, int q, CollectState& st)
{
    const int cntq = __builtin_amdgcn_readlane(st.cnt, q);
    const int64_t orow = static_cast<int64_t>(
        (static_cast<uint64_t>(static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(st.orow >> 32), q))) << 32) |
        static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(st.orow), q)));
    uint64_t* slots = a.cand + orow * kCollectCap;
    // the slots were stored by lanes q and q + 32: complete, then visible to
    // the wave (workgroup-scope loads)
    wait_vmem();
    wave_sync();
    constexpr int KPL = kCollectCap / 64;   // slots per lane
    static_assert(kCollectCap % 64 == 0, "whole slots per lane");
    uint64_t k[KPL];
#pragma unroll
    for (int i = 0; i < KPL; ++i)
        k[i] = lane + 64 * i < cntq
                   ? __hip_atomic_load(slots + lane + 64 * i, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP)
                   : kNoKey;
    // the M-th smallest key: the largest K with fewer than M keys below it
    const int M = a.M;
    uint64_t K = 0;
    for (int b = 63; b >= 0; --b) {
        const uint64_t t = K | (1ull << b);
        int below = 0;
#pragma unroll
        for (int i = 0; i < KPL; ++i) below += __popcll(__ballot(k[i] < t));
        if (below < M) K = t;
    }
    const uint64_t lt = (1ull << lane) - 1ull;
    int base = 0;
#pragma unroll
    for (int i = 0; i < KPL; ++i) {
        const bool p = k[i] <= K;
        const uint64_t m = __ballot(p);
        if (p) slots[base + __popcll(m & lt)] = k[i];
        base += __popcll(m);
    }
    if ((lane & 31) == q) {
        st.cnt = M;
        st.thr = o2f(static_cast<uint32_t>(K >> 32));
        st.thr_id = static_cast<uint32_t>(K);
    }
    if (a.stats && lane == 0) atomicAdd(a.stats + 1, 1ull);
}

// The query state the dense pass reads, published by lanes 0..31.
__device__ __forceinline__ void publish_state(CollectWave& W, int lane, bool qvalid, float qn, const CollectState& st)
{
    if (lane < kQueriesPerWave) {
        W.qst[lane] = make_float4(qn, qvalid ? st.thr : -INFINITY, __uint_as_float(st.thr_id), __int_as_float(st.self));
        W.qrow_out[lane] = st.orow;
    }
}

// One finished 32x32 tile of the collect scan: acc holds v = dot -
// floor(|p|^2 / 2) (L2) or dot (IP) for the pool rows with norms tn, ids tr
// and accumulator starts th (tile rows 8g + 4h + e in element 4g + e of lane
// (j, h)).  Tiles with no v at the lane's pass floor lo are dropped.  For the
// others the wave writes a code for every (lane, element) at or above the
// floor (a prefix sum of the lanes' counts places them), and then all 64
// lanes take one code each:
// the exact distance, the exact test against the query's (threshold, id)
// and the append to the query's slots (an LDS counter per query).  A query
// that could overflow its slots in this tile (more than kCollectCap - 32
// keys) is compacted first.
template <int METRIC>
__device__ __forceinline__ void collect_tile(const KnnArgs& a, CollectWave& W, const intx16& acc, const float* tn,
                                             const int32_t* tr, const int32_t* th, int lane, bool qvalid, float qn,
                                             CollectState& st, int32_t& lo)
{
    int32_t vmax = INT_MIN;
#pragma unroll
    for (int r = 0; r < 16; r += 2) vmax = max(vmax, max(acc[r], acc[r + 1]));
    if (!__ballot(vmax >= lo)) return;
    uint64_t need = __ballot(qvalid && st.cnt > kCollectCap - 2 * 16) & 0xffffffffull;
    if (need) {
        while (need) {
            const int q = __ffsll(static_cast<unsigned long long>(need)) - 1;
            need &= need - 1;
            collect_compact(a, lane, q, st);
        }
        lo = i8_pass_floor<METRIC>(st.thr, qn);
        publish_state(W, lane, qvalid, qn, st);
    }
#pragma unroll
    for (int c = 0; c < 4; ++c)
        *reinterpret_cast<int4*>(&W.stash[stash_index(lane, 4 * c)]) =
            make_int4(acc[4 * c], acc[4 * c + 1], acc[4 * c + 2], acc[4 * c + 3]);
    if (lane < kQueriesPerWave) W.qcnt[lane] = st.cnt;
    // codes in lane order, branch-free: each lane's candidates go to
    // [its exclusive prefix, + its count), the other elements to the lane's
    // spare slot
    int c = 0;
#pragma unroll
    for (int r = 0; r < 16; ++r) c += acc[r] >= lo ? 1 : 0;
    const int incl = wave_incl_scan(c);
    const int total = __builtin_amdgcn_readlane(incl, 63);
    int pos = incl - c;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
        const bool p = acc[r] >= lo;
        W.code[p ? pos : kCodeSpare + lane] = static_cast<uint16_t>((lane << 4) | r);
        pos += p ? 1 : 0;
    }
    wave_sync();
    for (int k = lane; k - lane < total; k += 64) {
        if (k < total) {
            const int code = W.code[k];
            const int src = code >> 4, r = code & 15;
            const int v = W.stash[stash_index(src, r)];
            const int q = src & 31;
            const int row = 8 * (r >> 2) + 4 * (src >> 5) + (r & 3);
            const float pn = tn[row];
            const int32_t id = tr[row];
            const int32_t hv = th[row];
            const float4 Q = W.qst[q];
            const float dot = static_cast<float>(v - hv);
            const float d = METRIC == 0 ? fmaf(-2.f, dot, pn + Q.x) : fmaf(-1.f, dot, pn);
            const bool ok = id >= 0 && id != __float_as_int(Q.w) &&
                            (d < Q.y || (d == Q.y && static_cast<uint32_t>(id) <= __float_as_uint(Q.z)));
            if (ok) {
                const int slot = atomicAdd(&W.qcnt[q], 1);
                a.cand[W.qrow_out[q] * kCollectCap + slot] = pack_key(d, id);
            }
        }
    }
    wave_sync();
    st.cnt = W.qcnt[lane & 31];
}

// The window pass's share of one finished tile: the lane's 16 distances
// (the query itself and rows past the slice end at +inf) join its sorted 32
// smallest.
template <int METRIC>
__device__ __forceinline__ void window_tile(const intx16& acc, const float* tn, const int32_t* tr, const int32_t* th,
                                            int h, float qn, int32_t self, float (&T)[32])
{
    float s[16];
#pragma unroll
    for (int g = 0; g < 4; ++g) {
        const float4 pn = *reinterpret_cast<const float4*>(tn + 8 * g + 4 * h);
        const int4 pi = *reinterpret_cast<const int4*>(tr + 8 * g + 4 * h);
        const int4 hv = *reinterpret_cast<const int4*>(th + 8 * g + 4 * h);
        const float n4[4] = {pn.x, pn.y, pn.z, pn.w};
        const int32_t i4[4] = {pi.x, pi.y, pi.z, pi.w};
        const int32_t h4[4] = {hv.x, hv.y, hv.z, hv.w};
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const float dot = static_cast<float>(acc[4 * g + e] - h4[e]);
            const float d = METRIC == 0 ? fmaf(-2.f, dot, n4[e] + qn) : fmaf(-1.f, dot, n4[e]);
            s[4 * g + e] = (i4[e] < 0 || i4[e] == self) ? INFINITY : d;
        }
    }
    oddeven_sort(s);
#pragma unroll
    for (int k = 0; k < 16; ++k) T[16 + k] = fminf(T[16 + k], s[15 - k]);
    bitonic_merge(T);
}

template <int DP, int METRIC>
__global__ void __attribute__((amdgpu_flat_work_group_size(256, 256), amdgpu_waves_per_eu(3)))
knn_i8_collect_kernel(KnnArgs a)
{
    constexpr int KS = DP / 32;                     // MFMA steps per tile
    constexpr int U4_ROW = DP / 16;                 // 16-byte pieces per row
    constexpr int ROWS = kStageRows;
    constexpr int U4_STAGE = ROWS * U4_ROW;
    constexpr int U4_THREAD = (U4_STAGE + 255) / 256;
    static_assert(DP % 32 == 0, "row stride must be a multiple of 32 bytes");
    static_assert(ROWS <= 256 && kWindow % kStageTiles == 0 && kWindowMax % kStageTiles == 0, "stage shape");
    __shared__ CollectSmem<DP> sm;

    const int per = a.n_items / 8;
    const int item_idx = static_cast<int>(blockIdx.x % 8) * per + static_cast<int>(blockIdx.x / 8);
    if (item_idx >= a.n_items) return;
    const WorkItem it = a.items[item_idx];
    if (it.q_count <= 0) return;

    const int tid = threadIdx.x;
    const int w = tid >> 6, lane = tid & 63, j = lane & 31, h = lane >> 5;
    const int qlocal = w * kQueriesPerWave + j;
    const bool qvalid = qlocal < it.q_count;
    const int64_t qi = it.q_begin + qlocal;
    const int32_t qrow = qvalid ? (a.q_rows ? a.q_rows[qi] : static_cast<int32_t>(qi)) : 0;
    const float qn = (qvalid && METRIC == 0) ? a.nq[qrow] : 0.f;

    CollectState st;
    float seed = FLT_MAX;
    // the seed is read from the output row (the query row unless the item has an out_base)
    const int64_t orow_seed = it.out_base >= 0 ? it.out_base + qlocal : static_cast<int64_t>(qrow);
    if (qvalid && a.seed_d) seed = fminf(a.seed_d[orow_seed * a.seed_ld + a.seed_ld - 1], FLT_MAX);
    st.thr = qvalid ? seed : -INFINITY;
    st.thr_id = 0xffffffffu;
    st.cnt = 0;
    st.self = a.exclude_self ? qrow : -2;
    st.orow = it.out_base >= 0 ? it.out_base + qlocal : static_cast<int64_t>(qrow);
    if (it.p_count <= 0) {   // an empty pool: no candidates (the stage loads below need a row)
        if (qvalid && h == 0) a.cand_cnt[st.orow] = 0;
        return;
    }

    intx4 qf[KS];
    {
        const int8_t* qsrc = a.Xq8 + static_cast<int64_t>(qrow) * DP + 16 * h;   // qrow 0 if invalid
#pragma unroll
        for (int s = 0; s < KS; ++s) {
            const intx4 v = *reinterpret_cast<const intx4*>(qsrc + 32 * s);
#pragma unroll
            for (int e = 0; e < 4; ++e) qf[s][e] = qvalid ? v[e] : 0;
        }
    }

    CollectWave& W = sm.wv[w];
    publish_state(W, lane, qvalid, qn, st);

    // stages of ROWS pool rows; unseeded, the first nws stages bound the
    // threshold and are scanned again at the end
    const int pcount = it.p_count;
    const int nps = (pcount + ROWS - 1) / ROWS;
    const int nws = a.seed_d ? 0 : min(window_tiles(a) / kStageTiles, nps);
    const int nst = nps + nws;
    // Chunk pruning (L2, integer rows): once every query of the block has its
    // threshold, a stage is scanned only if some query may hold a key in it:
    // with c a chunk's centre and r >= the distance of its rows from c, a row
    // p of the chunk has |q - p| >= |q - c| - r, so a query with
    // |q - c| > r + sqrt(thr) has no key at or below thr there.  The steps
    // after the window follow the schedule sm.slist (the first two, already
    // requested during the window, unconditionally).
    const int nch = (pcount + kChunkRows - 1) / kChunkRows;
    const bool prune = METRIC == 0 && a.ch8 != nullptr && nch <= kMaxChunkWords * 32;
    int nsteps = nst;     // steps of the scan (stages, in schedule order)
    bool listed = false;  // the steps from nws on follow sm.slist
    // The pool list is the caller's (launch_knn_collect_select requires one).
    auto pool_pos = [&](int p) __attribute__((always_inline)) -> int64_t {
        p = min(p, pcount - 1) + it.p_rot;
        if (p >= pcount) p -= pcount;
        return it.p_begin + p;
    };
    auto stage_base = [&](int s) __attribute__((always_inline)) { return (s < nps ? s : s - nps) * ROWS; };
    // the stage scanned at step k (-1: none)
    auto sched = [&](int k) __attribute__((always_inline)) -> int {
        if (k >= nsteps) return -1;
        return (!listed || k < nws) ? k : static_cast<int>(sm.slist[k - nws]);
    };

    // fixed-size register sets indexed only by unrolled loop counters
    struct Rows {
        intx4 v[U4_THREAD];   // vector type: register moves, not aggregate copies
    } pre;
    // The threads < ROWS fetch their stage row's pool id (one stage ahead)
    // and norm; the ids reach every thread's row requests through LDS.
    const int r_own = tid & (ROWS - 1);
    auto stage_id = [&](int k, bool& valid) __attribute__((always_inline)) -> int32_t {
        const int s = sched(k);
        const int base = s >= 0 ? stage_base(s) : 0;
        valid = s >= 0 && base + r_own < pcount;
        return a.p_rows[pool_pos(base + r_own)];
    };
    auto load_rows = [&](const int32_t* ids) __attribute__((always_inline)) {
        static_for<0, U4_THREAD>([&](auto U) __attribute__((always_inline)) {
            const int e = min(tid + 256 * U.value, U4_STAGE - 1);
            pre.v[U.value] =
                *reinterpret_cast<const intx4*>(a.Xp8 + static_cast<int64_t>(ids[e / U4_ROW]) * DP + 16 * (e % U4_ROW));
        });
    };
    auto store_rows = [&](int buf) __attribute__((always_inline)) {
        static_for<0, U4_THREAD>([&](auto U) __attribute__((always_inline)) {
            const int e = tid + 256 * U.value;
            if (e < U4_STAGE) *reinterpret_cast<intx4*>(&sm.tile[buf][e / U4_ROW][16 * (e % U4_ROW)]) = pre.v[U.value];
        });
    };

    // The block's schedule: each wave marks the chunks some query of it may
    // need (centres staged through tile[0], 32 x 32 MFMA tiles of q.c), the
    // marks are ORed over the waves, and wave 0 lists the stages from
    // `from` on that touch a marked chunk (stages before `first_free`
    // unconditionally).  Called by every thread; tile[0], tnorm[0..1] are free.
    auto build_schedule = [&](int from, int first_free) __attribute__((always_inline)) {
        __syncthreads();   // every wave is done with tile[0] and the norm slots
        const float sthr = st.thr >= 0.f ? sqrtf(st.thr) : -1.f;   // -1: the query needs nothing (invalid)
        const bool qneed = qvalid && sthr >= 0.f;
        for (int cb = 0; cb < nch; cb += ROWS) {
            const int nc = min(ROWS, nch - cb);
            static_for<0, U4_THREAD>([&](auto U) __attribute__((always_inline)) {
                const int e = tid + 256 * U.value;
                if (e < U4_STAGE) {
                    const int r = e / U4_ROW;
                    const int g = min(r, nc - 1);
                    *reinterpret_cast<intx4*>(&sm.tile[0][r][16 * (e % U4_ROW)]) = *reinterpret_cast<const intx4*>(
                        a.ch8 + (static_cast<int64_t>(it.p_begin / kChunkRows) + cb + g) * DP + 16 * (e % U4_ROW));
                }
            });
            if (tid < ROWS) {
                const int64_t g = it.p_begin / kChunkRows + cb + min(tid, nc - 1);
                sm.tnorm[0][tid] = a.chn[g];
                sm.tnorm[1][tid] = a.chr[g];
            }
            __syncthreads();
#pragma unroll
            for (int u = 0; u < kStageTiles; ++u) {
                intx16 acc;
#pragma unroll
                for (int r = 0; r < 16; ++r) acc[r] = 0;
                const int8_t* arow = &sm.tile[0][kPoolTile * u + j][16 * h];
#pragma unroll
                for (int k = 0; k < KS; ++k) {
                    const intx4 av = *reinterpret_cast<const intx4*>(arow + 32 * k);
                    acc = __builtin_amdgcn_mfma_i32_32x32x32_i8(av, qf[k], acc, 0, 0, 0);
                }
                uint32_t word = 0u;
#pragma unroll
                for (int g = 0; g < 4; ++g) {
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        const int row = kPoolTile * u + 8 * g + 4 * h + e;   // this lane's chunk (in the batch)
                        const float dqc = qn + sm.tnorm[0][row] - 2.f * static_cast<float>(acc[4 * g + e]);
                        const float lim = sm.tnorm[1][row] + sthr;
                        const bool need = qneed && cb + row < nch && dqc <= fmaf(lim, lim, 1.f) * 1.000001f;
                        const uint64_t bal = __ballot(need);
                        word |= ((bal & 0xffffffffull) != 0 ? 1u : 0u) << (8 * g + e);
                        word |= ((bal >> 32) != 0 ? 1u : 0u) << (8 * g + 4 + e);
                    }
                }
                if (lane == 0) sm.wmask[w][(cb + kPoolTile * u) / 32] = word;
            }
            __syncthreads();   // tile[0] and tnorm are read before the next batch
        }
        if (tid < (nch + 31) / 32)
            sm.bmask[tid] = sm.wmask[0][tid] | sm.wmask[1][tid] | sm.wmask[2][tid] | sm.wmask[3][tid];
        __syncthreads();
        if (w == 0) {
            const uint64_t lt = (1ull << lane) - 1ull;
            int n = 0;
            for (int s0 = from; s0 < nst; s0 += 64) {
                const int s = s0 + lane;
                bool need = false;
                if (s < nst) {
                    if (s < first_free) {
                        need = true;
                    } else {
                        // the chunks of the stage's first and last positions (a
                        // stage wrapping past the pool's end touches both ends)
                        const int base = stage_base(s);
                        const int p0 = static_cast<int>(pool_pos(base) - it.p_begin);
                        const int p1 = static_cast<int>(pool_pos(min(base + ROWS - 1, pcount - 1)) - it.p_begin);
                        const int c0 = p0 / kChunkRows, c1 = p1 / kChunkRows;
                        auto bit = [&](int c) { return (sm.bmask[c >> 5] >> (c & 31)) & 1u; };
                        if (c0 <= c1) {
                            for (int c = c0; c <= c1; ++c) need |= bit(c) != 0u;
                        } else {
                            for (int c = c0; c < nch; ++c) need |= bit(c) != 0u;
                            for (int c = 0; c <= c1; ++c) need |= bit(c) != 0u;
                        }
                    }
                }
                const uint64_t m = __ballot(need);
                if (need) sm.slist[n + __popcll(m & lt)] = static_cast<uint16_t>(s);
                n += __popcll(m);
            }
            if (lane == 0) sm.nlist = n;
        }
        __syncthreads();
        nsteps = from + sm.nlist;
        listed = true;
    };
    if (prune && nws == 0) build_schedule(0, 0);   // seeded: the thresholds are known

    int32_t rid_cur = 0, rid_next = 0;   // threads < ROWS: the stage row's id (a valid row) this stage, the next
    bool rvalid_cur = false, rvalid_next = false;
    float rn_cur = 0.f;
    if (tid < ROWS) {
        rid_cur = stage_id(0, rvalid_cur);
        sm.sid[0][tid] = rid_cur;
        rn_cur = METRIC == 0 ? a.np[rid_cur] : 0.f;
        rid_next = stage_id(1, rvalid_next);
    }
    __syncthreads();
    load_rows(sm.sid[0]);

    intx16 acc_prev;
#pragma unroll
    for (int r = 0; r < 16; ++r) acc_prev[r] = 0;
    int32_t lo = i8_pass_floor<METRIC>(st.thr, qn);
    bool pending = false;   // acc_prev holds tile p_u of step p_k, not yet filtered
    int p_k = 0, p_u = 0;

    // one step k: its stage's rows and norms (requested one step earlier)
    // into LDS, the barrier, the requests for step k + 1 (and the pool ids of
    // k + 2), then the MFMAs of the stage's tiles, each with filt on the tile
    // before it.  A request is waited for only at the next step's top, a
    // whole stage of MFMAs and filtering later.
    auto stage = [&](int k, auto&& filt) __attribute__((always_inline)) {
        const int buf = k & 1, slot = k % 3;
        store_rows(buf);
        if (tid < ROWS) {
            // rows past the slice end: id -1, norm +inf, accumulator start
            // kHalfPast keep them out of every result
            sm.trow[slot][tid] = rvalid_cur ? rid_cur : -1;
            sm.tnorm[slot][tid] = rvalid_cur ? rn_cur : INFINITY;
            sm.thalf[slot][tid] = rvalid_cur ? -(static_cast<int32_t>(rn_cur) >> 1) : kHalfPast;
            sm.sid[(k + 1) & 1][tid] = rid_next;
        }
        __syncthreads();
        load_rows(sm.sid[(k + 1) & 1]);
        if (tid < ROWS) {
            rid_cur = rid_next;
            rvalid_cur = rvalid_next;
            rn_cur = METRIC == 0 ? a.np[rid_cur] : 0.f;
            rid_next = stage_id(k + 2, rvalid_next);
        }

#pragma unroll
        for (int u = 0; u < kStageTiles; ++u) {
            intx16 acc;
            {
                const int32_t* th = &sm.thalf[slot][kPoolTile * u];
#pragma unroll
                for (int g = 0; g < 4; ++g) {
                    const int4 hv = *reinterpret_cast<const int4*>(th + 8 * g + 4 * h);
                    acc[4 * g] = hv.x; acc[4 * g + 1] = hv.y; acc[4 * g + 2] = hv.z; acc[4 * g + 3] = hv.w;
                }
            }
            const int8_t* arow = &sm.tile[buf][kPoolTile * u + j][16 * h];
#pragma unroll
            for (int kk = 0; kk < KS; ++kk) {
                const intx4 av = *reinterpret_cast<const intx4*>(arow + 32 * kk);
                acc = __builtin_amdgcn_mfma_i32_32x32x32_i8(av, qf[kk], acc, 0, 0, 0);
            }
            if (pending) filt(p_k, p_u);
            acc_prev = acc;
            pending = true;
            p_k = k;
            p_u = u;
        }
    };
    auto collect = [&](int k, int u) __attribute__((always_inline)) {
        const int slot = k % 3;
        collect_tile<METRIC>(a, W, acc_prev, &sm.tnorm[slot][kPoolTile * u], &sm.trow[slot][kPoolTile * u],
                             &sm.thalf[slot][kPoolTile * u], lane, qvalid, qn, st, lo);
    };
    if (nws > 0) {
        float T[32];
#pragma unroll
        for (int i = 0; i < 32; ++i) T[i] = INFINITY;
        auto window = [&](int k, int u) __attribute__((always_inline)) {
            const int slot = k % 3;
            window_tile<METRIC>(acc_prev, &sm.tnorm[slot][kPoolTile * u], &sm.trow[slot][kPoolTile * u],
                                &sm.thalf[slot][kPoolTile * u], h, qn, st.self, T);
        };
        for (int k = 0; k < nws; ++k) stage(k, window);
        window(p_k, p_u);   // the window's last tile
        pending = false;
        // the pair's ceil(M/2)-th smallest distances: M distinct rows at or below the larger
        const int m = (a.M + 1) / 2 - 1;
        float v = T[0];
#pragma unroll
        for (int i = 1; i < 32; ++i) v = i == m ? T[i] : v;
        const float bound = fmaxf(v, __shfl_xor(v, 32));
        if (qvalid && bound < st.thr) st.thr = bound;
        lo = i8_pass_floor<METRIC>(st.thr, qn);
        publish_state(W, lane, qvalid, qn, st);
        // the steps nws and nws + 1 are requested already: they stay
        if (prune) build_schedule(nws, nws + 2);
    }
    for (int k = nws; k < nsteps; ++k) stage(k, collect);
    if (pending) collect(p_k, p_u);
    if (qvalid && h == 0) a.cand_cnt[st.orow] = st.cnt;
    if (a.stats && qvalid && h == 0) atomicAdd(a.stats, static_cast<unsigned long long>(st.cnt));
    if (a.pairs_done && tid == 0)
        atomicAdd(a.pairs_done, static_cast<unsigned long long>(nsteps) * ROWS * static_cast<unsigned>(it.q_count));
}

// ------------------------------------------------------------ fp32 rows
//
// knn_f32_collect_kernel: the same collect scan on fp32 rows (float data,
// Dp <= 160).  Its distances are the merging fp32 kernel's (knn_fused_kernel)
// bit for bit -- the same v_mfma_f32_32x32x2_f32 chain per 32x32 tile
// (accumulator from 0, dimensions in the same order, lane (j, h) holding
// dims [h Dp/2, h Dp/2 + Dp/2) of query j) and the same key
// fmaf(-2, dot, |p|^2 + |q|^2) (L2) or -dot (IP) -- so the selected lists
// equal the merging kernel's.  One 32-row pool tile per step, double-buffered
// in LDS as in knn_fused_kernel (a tile is Dp/2 MFMAs per wave, long enough
// to hide the next tile's loads); rows past the slice end have norm +inf.

template <int DP>
struct CollectSmemF {
    float tile[2][kPoolTile][DP + 4];   // +4 floats: rows land on distinct bank groups
    float tnorm[3][kPoolTile];
    int32_t trow[3][kPoolTile];
    int32_t sid[2][kPoolTile];   // the next tile's pool row ids (-1 past the end), for every thread's row requests
    CollectWave wv[kWaves];
};

// The lane's 16 keys of a finished tile (pool row 8g + 4h + e in element
// 4g + e; rows past the slice end +inf).
template <int METRIC>
__device__ __forceinline__ void f32_tile_keys(const floatx16& acc, const float* tn, int h, float qn, float (&d)[16])
{
#pragma unroll
    for (int g = 0; g < 4; ++g) {
        const float4 pn = *reinterpret_cast<const float4*>(tn + 8 * g + 4 * h);
        const float n4[4] = {pn.x, pn.y, pn.z, pn.w};
#pragma unroll
        for (int e = 0; e < 4; ++e)
            d[4 * g + e] = METRIC == 0 ? fmaf(-2.f, acc[4 * g + e], n4[e] + qn) : fmaf(-1.f, acc[4 * g + e], n4[e]);
    }
}

// collect_tile for fp32 keys: the stash holds the keys themselves; a code is
// written for every key at or below the query's threshold, and the exact
// (key, id) test and the append are made per code.
template <int METRIC>
__device__ __forceinline__ void collect_tile_f32(const KnnArgs& a, CollectWave& W, const floatx16& acc,
                                                 const float* tn, const int32_t* tr, int lane, int h, bool qvalid,
                                                 float qn, CollectState& st)
{
    float d[16];
    f32_tile_keys<METRIC>(acc, tn, h, qn, d);
    float dmin = d[0];
#pragma unroll
    for (int r = 1; r < 16; ++r) dmin = fminf(dmin, d[r]);
    if (!__ballot(dmin <= st.thr)) return;
    uint64_t need = __ballot(qvalid && st.cnt > kCollectCap - 2 * 16) & 0xffffffffull;
    if (need) {
        while (need) {
            const int q = __ffsll(static_cast<unsigned long long>(need)) - 1;
            need &= need - 1;
            collect_compact(a, lane, q, st);
        }
        publish_state(W, lane, qvalid, qn, st);
    }
#pragma unroll
    for (int c = 0; c < 4; ++c)
        *reinterpret_cast<int4*>(&W.stash[stash_index(lane, 4 * c)]) =
            make_int4(__float_as_int(d[4 * c]), __float_as_int(d[4 * c + 1]), __float_as_int(d[4 * c + 2]),
                      __float_as_int(d[4 * c + 3]));
    if (lane < kQueriesPerWave) W.qcnt[lane] = st.cnt;
    int c = 0;
#pragma unroll
    for (int r = 0; r < 16; ++r) c += d[r] <= st.thr ? 1 : 0;
    const int incl = wave_incl_scan(c);
    const int total = __builtin_amdgcn_readlane(incl, 63);
    int pos = incl - c;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
        const bool p = d[r] <= st.thr;
        W.code[p ? pos : kCodeSpare + lane] = static_cast<uint16_t>((lane << 4) | r);
        pos += p ? 1 : 0;
    }
    wave_sync();
    for (int k = lane; k - lane < total; k += 64) {
        if (k < total) {
            const int code = W.code[k];
            const int src = code >> 4, r = code & 15;
            const float dk = __int_as_float(W.stash[stash_index(src, r)]);
            const int q = src & 31;
            const int row = 8 * (r >> 2) + 4 * (src >> 5) + (r & 3);
            const int32_t id = tr[row];
            const float4 Q = W.qst[q];
            const bool ok = id >= 0 && id != __float_as_int(Q.w) &&
                            (dk < Q.y || (dk == Q.y && static_cast<uint32_t>(id) <= __float_as_uint(Q.z)));
            if (ok) {
                const int slot = atomicAdd(&W.qcnt[q], 1);
                a.cand[W.qrow_out[q] * kCollectCap + slot] = pack_key(dk, id);
            }
        }
    }
    wave_sync();
    st.cnt = W.qcnt[lane & 31];
}

// window_tile for fp32 keys.
template <int METRIC>
__device__ __forceinline__ void window_tile_f32(const floatx16& acc, const float* tn, const int32_t* tr, int h,
                                                float qn, int32_t self, float (&T)[32])
{
    float s[16];
    f32_tile_keys<METRIC>(acc, tn, h, qn, s);
#pragma unroll
    for (int g = 0; g < 4; ++g) {
        const int4 pi = *reinterpret_cast<const int4*>(tr + 8 * g + 4 * h);
        const int32_t i4[4] = {pi.x, pi.y, pi.z, pi.w};
#pragma unroll
        for (int e = 0; e < 4; ++e) s[4 * g + e] = (i4[e] < 0 || i4[e] == self) ? INFINITY : s[4 * g + e];
    }
    oddeven_sort(s);
#pragma unroll
    for (int k = 0; k < 16; ++k) T[16 + k] = fminf(T[16 + k], s[15 - k]);
    bitonic_merge(T);
}

template <int DP, int METRIC>
__global__ void __launch_bounds__(256, 2) knn_f32_collect_kernel(KnnArgs a)
{
    constexpr int DH = DP / 2;                       // k-steps of 2 dims (one per half wave)
    constexpr int F4_ROW = DP / 4;
    constexpr int F4_THREAD = kPoolTile * F4_ROW / 256;
    static_assert(DP % 32 == 0, "row stride must be a multiple of 32 floats");
    __shared__ CollectSmemF<DP> sm;

    const int per = a.n_items / 8;
    const int item_idx = static_cast<int>(blockIdx.x % 8) * per + static_cast<int>(blockIdx.x / 8);
    if (item_idx >= a.n_items) return;
    const WorkItem it = a.items[item_idx];
    if (it.q_count <= 0) return;

    const int tid = threadIdx.x;
    const int w = tid >> 6, lane = tid & 63, j = lane & 31, h = lane >> 5;
    const int qlocal = w * kQueriesPerWave + j;
    const bool qvalid = qlocal < it.q_count;
    const int64_t qi = it.q_begin + qlocal;
    const int32_t qrow = qvalid ? (a.q_rows ? a.q_rows[qi] : static_cast<int32_t>(qi)) : 0;
    const float qn = (qvalid && METRIC == 0) ? a.nq[qrow] : 0.f;

    CollectState st;
    float seed = FLT_MAX;
    const int64_t orow_seed = it.out_base >= 0 ? it.out_base + qlocal : static_cast<int64_t>(qrow);
    if (qvalid && a.seed_d) seed = fminf(a.seed_d[orow_seed * a.seed_ld + a.seed_ld - 1], FLT_MAX);
    st.thr = qvalid ? seed : -INFINITY;
    st.thr_id = 0xffffffffu;
    st.cnt = 0;
    st.self = a.exclude_self ? qrow : -2;
    st.orow = it.out_base >= 0 ? it.out_base + qlocal : static_cast<int64_t>(qrow);

    // query fragment: dims [h*DH, h*DH + DH) of query row qrow
    float qf[DH];
    {
        const float4* src = reinterpret_cast<const float4*>(a.Xq + static_cast<int64_t>(qrow) * DP + h * DH);
#pragma unroll
        for (int s4 = 0; s4 < DH / 4; ++s4) {
            const float4 v = qvalid ? src[s4] : make_float4(0.f, 0.f, 0.f, 0.f);
            qf[4 * s4 + 0] = v.x; qf[4 * s4 + 1] = v.y; qf[4 * s4 + 2] = v.z; qf[4 * s4 + 3] = v.w;
        }
    }

    CollectWave& W = sm.wv[w];
    publish_state(W, lane, qvalid, qn, st);

    // steps: tiles 0 .. ntl - 1, each once; unseeded, the first nwt tiles
    // bound the threshold first and are scanned again at the end
    const int pcount = it.p_count;
    const int ntl = (pcount + kPoolTile - 1) / kPoolTile;
    const int nwt = a.seed_d ? 0 : min(window_tiles(a), ntl);
    const int nst = ntl + nwt;
    auto pool_row = [&](int t, int r) __attribute__((always_inline)) -> int32_t {
        if (t >= nst) return -1;
        int p = (t < ntl ? t : t - ntl) * kPoolTile + r;
        if (p >= pcount) return -1;
        p += it.p_rot;
        if (p >= pcount) p -= pcount;
        return a.p_rows[it.p_begin + p];
    };
    auto row_norm = [&](int32_t row) __attribute__((always_inline)) -> float {
        if (row < 0) return INFINITY;
        return METRIC == 0 ? a.np[row] : 0.f;
    };
    // pool tiles flow through three stages as in knn_fused_kernel: ids (two
    // steps ahead, one per row by the threads < kPoolTile, handed to every
    // thread through LDS) -> rows in registers (one step ahead) -> LDS
    float4 pre[F4_THREAD];
    int32_t rid_next = -1;   // threads < kPoolTile: the row id two tiles ahead
    auto load_rows = [&](const int32_t* ids) __attribute__((always_inline)) {
#pragma unroll
        for (int u = 0; u < F4_THREAD; ++u) {
            const int e = tid + 256 * u;
            const int32_t id = ids[e / F4_ROW];
            pre[u] = id >= 0 ? reinterpret_cast<const float4*>(a.Xp + static_cast<int64_t>(id) * DP)[e % F4_ROW]
                             : make_float4(0.f, 0.f, 0.f, 0.f);
        }
    };
    auto store_rows = [&](int buf) __attribute__((always_inline)) {
#pragma unroll
        for (int u = 0; u < F4_THREAD; ++u) {
            const int e = tid + 256 * u;
            *reinterpret_cast<float4*>(&sm.tile[buf][e / F4_ROW][4 * (e % F4_ROW)]) = pre[u];
        }
    };

    int32_t rid_cur = -1;
    float rn_cur = 0.f;
    if (tid < kPoolTile) {
        rid_cur = pool_row(0, tid);
        sm.sid[0][tid] = rid_cur;
        rn_cur = row_norm(rid_cur);
        rid_next = pool_row(1, tid);
    }
    __syncthreads();
    load_rows(sm.sid[0]);
    store_rows(0);
    if (tid < kPoolTile) { sm.trow[0][tid] = rid_cur; sm.tnorm[0][tid] = rn_cur; sm.sid[1][tid] = rid_next; }
    __syncthreads();

    floatx16 acc_prev;
#pragma unroll
    for (int r = 0; r < 16; ++r) acc_prev[r] = 0.f;
    bool pending = false;   // acc_prev holds step p_t's tile, not yet filtered
    int p_t = 0;
    // one step: the next tile's rows requested, the MFMAs of tile t, the
    // filter of the tile before it, then tile t + 1 into the other buffer
    auto step = [&](int t, auto&& filt) __attribute__((always_inline)) {
        const int buf = t & 1;
        wait_vmem();
        load_rows(sm.sid[(t + 1) & 1]);
        if (tid < kPoolTile) {
            rid_cur = rid_next;
            rn_cur = row_norm(rid_cur);
            rid_next = pool_row(t + 2, tid);
        }
        floatx16 acc;
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[r] = 0.f;
        const float* arow = &sm.tile[buf][j][h * DH];
#pragma unroll
        for (int s4 = 0; s4 < DH / 4; ++s4) {
            const float4 av = *reinterpret_cast<const float4*>(arow + 4 * s4);
            acc = __builtin_amdgcn_mfma_f32_32x32x2f32(av.x, qf[4 * s4 + 0], acc, 0, 0, 0);
            acc = __builtin_amdgcn_mfma_f32_32x32x2f32(av.y, qf[4 * s4 + 1], acc, 0, 0, 0);
            acc = __builtin_amdgcn_mfma_f32_32x32x2f32(av.z, qf[4 * s4 + 2], acc, 0, 0, 0);
            acc = __builtin_amdgcn_mfma_f32_32x32x2f32(av.w, qf[4 * s4 + 3], acc, 0, 0, 0);
        }
        if (pending) filt(p_t);
        store_rows(buf ^ 1);
        if (tid < kPoolTile) {
            sm.trow[(t + 1) % 3][tid] = rid_cur;
            sm.tnorm[(t + 1) % 3][tid] = rn_cur;
            sm.sid[t & 1][tid] = rid_next;   // tile t + 2's ids
        }
        __syncthreads();
        acc_prev = acc;
        pending = true;
        p_t = t;
    };
    auto collect = [&](int t) __attribute__((always_inline)) {
        const int sl = t % 3;
        collect_tile_f32<METRIC>(a, W, acc_prev, sm.tnorm[sl], sm.trow[sl], lane, h, qvalid, qn, st);
    };
    if (nwt > 0) {
        float T[32];
#pragma unroll
        for (int i = 0; i < 32; ++i) T[i] = INFINITY;
        auto window = [&](int t) __attribute__((always_inline)) {
            const int sl = t % 3;
            window_tile_f32<METRIC>(acc_prev, sm.tnorm[sl], sm.trow[sl], h, qn, st.self, T);
        };
        for (int t = 0; t < nwt; ++t) step(t, window);
        window(p_t);   // the window's last tile
        pending = false;
        // the pair's ceil(M/2)-th smallest distances: M distinct rows at or below the larger
        const int m = (a.M + 1) / 2 - 1;
        float v = T[0];
#pragma unroll
        for (int i = 1; i < 32; ++i) v = i == m ? T[i] : v;
        const float bound = fmaxf(v, __shfl_xor(v, 32));
        if (qvalid && bound < st.thr) st.thr = bound;
        publish_state(W, lane, qvalid, qn, st);
    }
    for (int t = nwt; t < nst; ++t) step(t, collect);
    if (pending) collect(p_t);
    if (qvalid && h == 0) a.cand_cnt[st.orow] = st.cnt;
    if (a.stats && qvalid && h == 0) atomicAdd(a.stats, static_cast<unsigned long long>(st.cnt));
}

// ------------------------------------------------------------ selection

// Each row's top-M of its cnt[row] candidate keys, ascending, into (out_ids,
// out_d) (padding -1 / +inf).  Two lanes per row, 128 rows per block; lane
// (j, h) of a wave keeps positions LM h .. LM h + LM - 1 of row j's list.
// Rows with at most skip_le keys are neither selected nor written (-1: every
// row is).  LIST: the rows are rlist[0 .. *rcount) (output row i = list
// entry i).
// Keys and results move through a per-wave LDS stage so that every global
// access is whole rows: each of a wave's 8 loads per step brings 32 keys of
// 4 rows (16 lanes x 16 bytes per row), all 8 issued before the stage is
// written, and the wave's 32 output rows, contiguous in out_ids and out_d,
// leave as 16-byte stores.  `cand` must hold kQueriesPerWave rows of slack
// past the last row.  Staged rows are 34 keys (results: M + 4 words)
// apart, so that the 16 lanes of an LDS pass hit distinct banks.  (Loading
// the stage by LDS DMA, the next step's keys in flight during the merge,
// measured slower: the merges are VALU-bound and the DMA version fits two
// waves per SIMD instead of three.)
constexpr int kSelStride = 2 * 16 + 2;   // keys per staged row

template <int LM, bool LIST>
__global__ void __attribute__((amdgpu_flat_work_group_size(256, 256), amdgpu_waves_per_eu(LIST ? 2 : 3))) knn_select_kernel(const uint64_t* __restrict__ cand,
                                                         const int32_t* __restrict__ cnt, int64_t rows, int M,
                                                         int skip_le, const int32_t* __restrict__ rlist,
                                                         const uint32_t* __restrict__ rcount,
                                                         int32_t* __restrict__ out_ids, float* __restrict__ out_d)
{
    __shared__ __align__(16) uint64_t stage[kWaves][kQueriesPerWave * kSelStride];
    const int lane = threadIdx.x & 63, h = lane >> 5, j = lane & 31;
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    if (LIST) rows = __builtin_amdgcn_readfirstlane(static_cast<int>(*rcount));
    const int64_t row0 = (static_cast<int64_t>(blockIdx.x) * kWaves + w) * kQueriesPerWave;
    if (row0 >= rows) return;   // wave-uniform
    const int nrows = static_cast<int>(min(static_cast<int64_t>(kQueriesPerWave), rows - row0));
    // LIST: the table row of the wave's row j (the loads take row rq + 4 t's
    // from its lane)
    const int32_t lrow = LIST ? rlist[min(row0 + j, rows - 1)] : 0;
    const int n_all = j < nrows ? min(cnt[LIST ? static_cast<int64_t>(lrow) : row0 + j], kCollectCap) : 0;
    const bool valid = j < nrows && n_all > skip_le;
    const uint64_t vrows = __ballot(valid && h == 0);   // bit j: row j is written
    if (vrows == 0) return;                              // wave-uniform
    const int n = valid ? n_all : 0;
    uint64_t* st = stage[w];
    PairList<LM> PL;
#pragma unroll
    for (int i = 0; i < LM; ++i) PL.k[i] = kNoKey;
    const int q = lane & 15, rq = lane >> 4;
    // keys c0 .. c0 + 31 of every row of the wave into b (16 per lane)
    auto step = [&](int c0, uint64_t (&b)[16]) __attribute__((always_inline)) {
        // all 8 loads in flight before the stage is written: every lane loads
        // its 16 bytes of rows rq, rq + 4, ... whatever the rows' counts (the
        // keys past a count and the rows past the last are masked below; the
        // buffer holds a wave's rows of slack past the last row)
        const uint64_t* src = cand + (row0 + rq) * kCollectCap + c0 + 2 * q;
        intx4 x[8];   // vector type: kept in registers (an array of uint4 structs went to scratch)
#pragma unroll
        for (int t = 0; t < 8; ++t)
            x[t] = LIST ? *reinterpret_cast<const intx4*>(cand + static_cast<int64_t>(__shfl(lrow, rq + 4 * t)) * kCollectCap +
                                                          c0 + 2 * q)
                        : *reinterpret_cast<const intx4*>(src + 4 * t * kCollectCap);
        uint64_t* dst = st + rq * kSelStride + 2 * q;
#pragma unroll
        for (int t = 0; t < 8; ++t) *reinterpret_cast<intx4*>(dst + 4 * t * kSelStride) = x[t];
        wave_sync();
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const uint4 x = *reinterpret_cast<const uint4*>(st + j * kSelStride + 16 * h + 2 * e);
            const int i = c0 + 16 * h + 2 * e;
            b[2 * e] = i < n ? (static_cast<uint64_t>(x.y) << 32) | x.x : kNoKey;
            b[2 * e + 1] = i + 1 < n ? (static_cast<uint64_t>(x.w) << 32) | x.z : kNoKey;
        }
        wave_sync();   // the stage is read before the next step refills it
    };
    if (__ballot(n > 0)) {
        uint64_t b[16];
        step(0, b);
        pair_first32<LM>(b, PL, h != 0);
    }
    for (int c0 = 32; __ballot(c0 < n); c0 += 32) {
        uint64_t b[16];
        step(c0, b);
        pair_merge32<LM>(b, PL, h != 0);
    }
    // ids, then distances, through the stage (row stride Ms words)
    uint32_t* so = reinterpret_cast<uint32_t*>(st);
    const int Ms = (M + 3) / 4 * 4 + 4;
    const int total = nrows * M;
    for (int pass = 0; pass < 2; ++pass) {
        if (valid) {
#pragma unroll
            for (int i = 0; i < LM; ++i) {
                const int p = LM * h + i;
                if (p < M) {
                    const uint64_t k = PL.k[i];
                    so[j * Ms + p] = pass == 0 ? (k == kNoKey ? 0xFFFFFFFFu : static_cast<uint32_t>(k))
                                               : __float_as_uint(k == kNoKey ? INFINITY
                                                                             : o2f(static_cast<uint32_t>(k >> 32)));
                }
            }
        }
        wave_sync();
        uint32_t* dst = pass == 0 ? reinterpret_cast<uint32_t*>(out_ids + row0 * M)
                                  : reinterpret_cast<uint32_t*>(out_d + row0 * M);
        if (M % 4 == 0) {
            for (int v = 4 * lane; v < total; v += 256) {
                const int r = v / M, p = v - r * M;
                if ((vrows >> r) & 1)
                    *reinterpret_cast<uint4*>(dst + v) = *reinterpret_cast<const uint4*>(so + r * Ms + p);
            }
        } else {
            for (int v = lane; v < total; v += 64) {
                const int r = v / M;
                if ((vrows >> r) & 1) dst[v] = so[r * Ms + (v - r * M)];
            }
        }
        wave_sync();   // read out before the distances overwrite it
    }
}

// ------------------------------------------------------------ merge into the running table

// The cross-round merge (src/bucket.cu:5021-5053) of a seeded pass, in place:
// running row r (ascending by (distance, id), padding (-1, +inf) last)
// becomes the top-M by (distance, id) of itself and the row's new list, a new
// id already in it dropped -- the rule and arithmetic of merge_rounds_kernel,
// on the same two lists, so the table is the same bit for bit.  Only rows
// that received keys are read or written: the merge of a running row with an
// empty list is the row.  The new list of a row with at most rank_max (<= M)
// keys is its keys ascending (the selection's list of it), ranked here from
// the collect buffer; a row with more was selected into (sel_ids, sel_d) by
// knn_select_kernel (skip_le = rank_max).  With rlist, the rows are
// rlist[0 .. *rcount) and selected row i is list entry i's.  One wave per
// rpw (<= 64) rows: the rows with keys one after another, the next one's
// loads in flight during each merge.
__global__ void __launch_bounds__(256) knn_merge_run_kernel(const uint64_t* __restrict__ cand,
                                                            const int32_t* __restrict__ cnt, int64_t rows, int M,
                                                            int rpw, int rank_max, const int32_t* __restrict__ rlist,
                                                            const uint32_t* __restrict__ rcount,
                                                            const int32_t* __restrict__ sel_ids,
                                                            const float* __restrict__ sel_d, int32_t* run_ids,
                                                            float* run_d)
{
    __shared__ float sRd[kWaves][64], sNd[kWaves][64];
    __shared__ int32_t sRi[kWaves][64], sNi[kWaves][64];
    __shared__ uint64_t sK[kWaves][64];
    const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
    if (rlist) rows = __builtin_amdgcn_readfirstlane(static_cast<int>(*rcount));
    const int64_t g0 = (static_cast<int64_t>(blockIdx.x) * kWaves + w) * rpw;
    if (g0 >= rows) return;   // wave-uniform
    // position g0 + lane's table row
    const bool mine = lane < rpw && g0 + lane < rows;
    const int32_t prow = mine ? (rlist ? rlist[g0 + lane] : static_cast<int32_t>(g0 + lane)) : 0;
    const int nl = mine ? min(cnt[prow], kCollectCap) : 0;
    uint64_t todo = __ballot(nl > 0);
    struct In {
        int32_t ri, ni;
        float rd, nd;
        uint64_t key;
    };
    // row g0 + r's running entry `lane`, and its new entry `lane` (selected
    // rows) or key `lane` (rows of at most M keys)
    auto load = [&](int r, In& x) __attribute__((always_inline)) {
        const int64_t row = __shfl(prow, r), srow = g0 + r;
        const int n = __shfl(nl, r);
        const bool in = lane < M;
        x.ri = in ? run_ids[row * M + lane] : -1;
        x.rd = in ? run_d[row * M + lane] : INFINITY;
        x.ni = -1;
        x.nd = INFINITY;
        x.key = kNoKey;
        if (n > rank_max) {
            if (in) {
                x.ni = sel_ids[srow * M + lane];
                x.nd = sel_d[srow * M + lane];
            }
        } else if (lane < n) {
            x.key = cand[row * kCollectCap + lane];
        }
    };
    if (todo == 0) return;
    int r = __builtin_ctzll(todo);
    In cur;
    load(r, cur);
    while (true) {
        todo &= todo - 1;
        const int rn = todo ? __builtin_ctzll(todo) : -1;
        In nxt;
        if (rn >= 0) load(rn, nxt);
        const int64_t row = __shfl(prow, r);
        const int n = __shfl(nl, r);
        int32_t niv = cur.ni;
        float ndv = cur.nd;
        if (n <= rank_max) {
            // the keys ascending: key q goes to its rank among the row's keys
            // (distinct: one key per pool row)
            sK[w][lane] = cur.key;
            wave_sync();
            int rank = 0;
            for (int q = 0; q < n; ++q) rank += sK[w][q] < cur.key ? 1 : 0;
            wave_sync();
            if (lane < n) sK[w][rank] = cur.key;
            wave_sync();
            const uint64_t k = sK[w][lane];
            const bool has = lane < n;
            niv = has ? static_cast<int32_t>(static_cast<uint32_t>(k)) : -1;
            ndv = has ? o2f(static_cast<uint32_t>(k >> 32)) : INFINITY;
        }
        // merge_rounds_kernel's steps for one row of at most 64 entries
        int32_t riv = cur.ri;
        const float rdv = riv >= 0 ? cur.rd : INFINITY;
        ndv = niv >= 0 ? ndv : INFINITY;
        if (riv < 0) riv = INT_MAX;
        sRd[w][lane] = rdv;
        sRi[w][lane] = riv;
        const int nr = static_cast<int>(__popcll(__ballot(riv != INT_MAX)));
        wave_sync();
        bool dup = false;
        if (niv >= 0)
            for (int q = 0; q < nr; ++q) dup |= (sRi[w][q] == niv);
        const bool keep = niv >= 0 && !dup;
        const unsigned long long below = lane == 0 ? 0ull : (~0ull >> (64 - lane));
        const unsigned long long km = __ballot(keep);
        const int nn = static_cast<int>(__popcll(km));
        const int cidx = static_cast<int>(__popcll(km & below));
        if (keep) {
            sNd[w][cidx] = ndv;
            sNi[w][cidx] = niv;
        }
        wave_sync();
        if (lane < nr) {
            const int pos = lane + lower_bound_g(sNd[w], sNi[w], nn, rdv, riv);
            if (pos < M) {
                run_ids[row * M + pos] = riv;
                run_d[row * M + pos] = rdv;
            }
        }
        if (keep) {
            const int pos = cidx + lower_bound_g(sRd[w], sRi[w], nr, ndv, niv);
            if (pos < M) {
                run_ids[row * M + pos] = niv;
                run_d[row * M + pos] = ndv;
            }
        }
        for (int p = nr + nn + lane; p < M; p += 64) {
            run_ids[row * M + p] = -1;
            run_d[row * M + p] = INFINITY;
        }
        wave_sync();   // the lists are read before the next row overwrites them
        if (rn < 0) break;
        r = rn;
        cur = nxt;
    }
}

// The same in-place merge for int8 rows, with the duplicates dropped before
// the top M is taken.  A pair's int8 distance is an exact integer, the same
// in every pass, so an id already in the running row comes back with the
// same key; and every key of a seeded pass lies at or below the row's
// running M-th distance, so the running row's own entries within the pass's
// pools come back (most of a later round's keys).  Dropping the keys whose
// ids the running row holds before taking the top M leaves the table of
// select-then-merge unchanged: a key outside the top M of the row's keys has
// M smaller keys, each in the running row or among the fresh ones.  Per row:
// the running ids go into two 256-slot LDS tables (slots by two multiplicative
// hashes); an id that lost both its slots to other ids is compared with the
// keys from registers (readlane), so a key's id is in the row iff a table
// slot or a lost id matches it; the fresh keys (at most kCollectCap) are
// ranked by counting and merged with merge_rounds_kernel's order and
// positions.  A row without fresh keys is not written; a row with more than
// M is left to the selection: appended to hl_rows (hl_count, zero on entry),
// for knn_select_kernel and knn_merge_run_kernel over that list.  Rows with
// keys are handled in order, RING rows' loads in flight.  The running table's
// distances must be the library's own (exact) ones.
constexpr int kFreshSlots = 256;
constexpr int kFreshRing = 2;   // rows in flight per wave of knn_merge_fresh_kernel
__device__ __forceinline__ int fresh_h1(int32_t id) { return static_cast<int>((static_cast<uint32_t>(id) * 0x9E3779B1u) >> 24); }
__device__ __forceinline__ int fresh_h2(int32_t id) { return static_cast<int>((static_cast<uint32_t>(id) * 0x85EBCA6Bu) >> 24); }

template <int RING>
__global__ void __launch_bounds__(256) knn_merge_fresh_kernel(const uint64_t* __restrict__ cand,
                                                              const int32_t* __restrict__ cnt, int64_t rows, int M,
                                                              int32_t* run_ids, float* run_d,
                                                              int32_t* __restrict__ hl_rows,
                                                              uint32_t* __restrict__ hl_count,
                                                              unsigned long long* __restrict__ stats)
{
    __shared__ int32_t sT1[kWaves][kFreshSlots], sT2[kWaves][kFreshSlots];
    __shared__ float sRd[kWaves][64], sNd[kWaves][64];
    __shared__ int32_t sRi[kWaves][64], sNi[kWaves][64];
    __shared__ uint64_t sF[kWaves][kCollectCap];
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
    const int64_t g0 = (static_cast<int64_t>(blockIdx.x) * kWaves + w) * 64;
    if (g0 >= rows) return;   // wave-uniform
    const int nl = g0 + lane < rows ? min(cnt[g0 + lane], kCollectCap) : 0;
    uint64_t todo = __ballot(nl > 0), heavy = 0;
    if (todo == 0) return;
    for (int i = lane; i < kFreshSlots; i += 64) {
        sT1[w][i] = -1;
        sT2[w][i] = -1;
    }
    struct In {
        int32_t ri;
        float rd;
        uint64_t key[4];   // keys lane, lane + 64, lane + 128, lane + 192
    };
    auto next = [&]() __attribute__((always_inline)) {
        if (todo == 0) return -1;
        const int r = __builtin_ctzll(todo);
        todo &= todo - 1;
        return r;
    };
    // a row's six loads are range-checked buffer loads based at the wave's
    // first row: a masked lane gets an offset past the range (it reads 0 and
    // fetches nothing), so every row issues the same loads without a branch
    // and the loads of the rows in flight are waited for one row at a time
    const int grows = static_cast<int>(min(static_cast<int64_t>(64), rows - g0));
    constexpr uint32_t kOut = 0x7FFFFFF0u;
    const __amdgpu_buffer_rsrc_t rs_i = __builtin_amdgcn_make_buffer_rsrc(run_ids + g0 * M, 0, grows * M * 4, 0x00020000);
    const __amdgpu_buffer_rsrc_t rs_d = __builtin_amdgcn_make_buffer_rsrc(run_d + g0 * M, 0, grows * M * 4, 0x00020000);
    const __amdgpu_buffer_rsrc_t rs_c = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint64_t*>(cand) + g0 * kCollectCap, 0, grows * kCollectCap * 8, 0x00020000);
    // (the raw words only: the masking is applied where the row is merged,
    // so that nothing waits for a row's loads before then)
    auto load = [&](int r, In& x) __attribute__((always_inline)) {
        if (r < 0) return;
        const int n = __shfl(nl, r);
        const uint32_t ro = lane < M ? static_cast<uint32_t>((r * M + lane) * 4) : kOut;
        x.ri = __builtin_amdgcn_raw_buffer_load_b32(rs_i, ro, 0, 0);
        x.rd = __int_as_float(__builtin_amdgcn_raw_buffer_load_b32(rs_d, ro, 0, 0));
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const uint32_t co = lane + 64 * j < n ? static_cast<uint32_t>((r * kCollectCap + lane + 64 * j) * 8) : kOut;
            const auto v = __builtin_amdgcn_raw_buffer_load_b64(rs_c, co, 0, 0);
            x.key[j] = (static_cast<uint64_t>(v[1]) << 32) | v[0];
        }
    };
    const unsigned long long below = lane == 0 ? 0ull : (~0ull >> (64 - lane));
    auto process = [&](int r, const In& raw) __attribute__((always_inline)) {
        const int64_t row = g0 + r;
        const int n = __shfl(nl, r);
        const int nk = (n + 63) >> 6;   // 64-key chunks holding keys (uniform)
        In cur;   // masked lanes: id -1 / distance +inf, key kNoKey (they read 0)
        cur.ri = lane < M ? raw.ri : -1;
        cur.rd = lane < M ? raw.rd : INFINITY;
#pragma unroll
        for (int j = 0; j < 4; ++j) cur.key[j] = lane + 64 * j < n ? raw.key[j] : kNoKey;
        int32_t riv = cur.ri;
        const float rdv = riv >= 0 ? cur.rd : INFINITY;
        if (riv < 0) riv = INT_MAX;
        const bool rv = riv != INT_MAX;
        const int nr = static_cast<int>(__popcll(__ballot(rv)));
        const int h1 = fresh_h1(riv), h2 = fresh_h2(riv);
        if (rv) {
            sT1[w][h1] = riv;
            sT2[w][h2] = riv;
        }
        sRd[w][lane] = rdv;
        sRi[w][lane] = riv;
        wave_sync();
        int32_t kid[4];
        bool held[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            kid[j] = static_cast<int32_t>(static_cast<uint32_t>(cur.key[j]));
            held[j] = false;
            if (j < nk) held[j] = (sT1[w][fresh_h1(kid[j])] == kid[j]) | (sT2[w][fresh_h2(kid[j])] == kid[j]);
        }
        // the running ids that lost both slots, compared from registers
        uint64_t lost = __ballot(rv & (sT1[w][h1] != riv) & (sT2[w][h2] != riv));
        while (lost) {
            const int l = __builtin_ctzll(lost);
            lost &= lost - 1;
            const int32_t id = __builtin_amdgcn_readlane(riv, l);
#pragma unroll
            for (int j = 0; j < 4; ++j)
                if (j < nk) held[j] |= kid[j] == id;
        }
        // fresh keys, compacted in slot order
        int f = 0;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            if (j >= nk) break;
            const bool fresh = (cur.key[j] != kNoKey) & !held[j];
            const unsigned long long fm = __ballot(fresh);
            if (fresh) sF[w][f + static_cast<int>(__popcll(fm & below))] = cur.key[j];
            f += static_cast<int>(__popcll(fm));
        }
        if (stats && lane == 0) {   // optional counters: [4] rows, [5] fresh keys, [6] rows with some, [7] > M
            atomicAdd(stats + 4, 1ull);
            atomicAdd(stats + 5, static_cast<unsigned long long>(f));
            if (f > 0) atomicAdd(stats + 6, 1ull);
            if (f > M) atomicAdd(stats + 7, 1ull);
        }
        wave_sync();
        sT1[w][h1] = -1;   // every slot written for this row back to empty (after the lookups above)
        sT2[w][h2] = -1;
        if (f == 0) return;
        if (f > M) {   // to the selection (listed when the wave ends)
            heavy |= 1ull << r;
            return;
        }
        // fresh key `lane`'s rank among the fresh keys (distinct)
        const uint64_t fk = lane < f ? sF[w][lane] : kNoKey;
        int rk = 0;
        for (int t = 0; t < f; ++t) rk += sF[w][t] < fk ? 1 : 0;
        if (lane < f) {
            sNd[w][rk] = o2f(static_cast<uint32_t>(fk >> 32));
            sNi[w][rk] = static_cast<int32_t>(static_cast<uint32_t>(fk));
        }
        const int nn = f;
        wave_sync();
        if (lane < nr) {
            const int pos = lane + lower_bound_g(sNd[w], sNi[w], nn, rdv, riv);
            if (pos < M) {
                run_ids[row * M + pos] = riv;
                run_d[row * M + pos] = rdv;
            }
        }
        if (lane < nn) {
            const float nd = sNd[w][lane];
            const int32_t ni = sNi[w][lane];
            const int pos = lane + lower_bound_g(sRd[w], sRi[w], nr, nd, ni);
            if (pos < M) {
                run_ids[row * M + pos] = ni;
                run_d[row * M + pos] = nd;
            }
        }
        for (int p = nr + nn + lane; p < M; p += 64) {
            run_ids[row * M + p] = -1;
            run_d[row * M + p] = INFINITY;
        }
        wave_sync();   // the lists are read before the next row overwrites them
    };
    // a ring of RING rows: a slot is refilled with the next row as soon as
    // its row is merged (rows leave todo in ascending order, so a slot
    // without a row means no row follows)
    In buf[RING];
    int rr[RING];
#pragma unroll
    for (int i = 0; i < RING; ++i) {
        rr[i] = next();
        load(rr[i], buf[i]);
    }
    bool more = true;
    while (more) {
#pragma unroll
        for (int i = 0; i < RING; ++i) {
            if (more && rr[i] < 0) more = false;
            if (more) {
                process(rr[i], buf[i]);
                rr[i] = next();
                load(rr[i], buf[i]);
            }
        }
    }
    // the wave's rows for the selection: one counter update per wave (one
    // per row serialised on the counter)
    if (heavy) {
        uint32_t base = 0;
        if (lane == 0) base = atomicAdd(hl_count, static_cast<uint32_t>(__popcll(heavy)));
        base = __shfl(base, 0);
        if ((heavy >> lane) & 1)
            hl_rows[base + static_cast<uint32_t>(__popcll(heavy & below))] = static_cast<int32_t>(g0 + lane);
    }
}

// Per pruning chunk g (pool-list rows [kChunkRows g, + cnt[g])): the
// rounded mean of its int8 rows as its centre c, |c|^2, and sqrt of the
// largest |p - c|^2 of its rows (exact integers; the root rounded up by a
// relative 2^-20), for knn_i8_collect_kernel's stage skipping (Dp a power
// of two, at most 256).  One wave per chunk, four chunks per block: lane l
// holds the 16-byte piece l % (Dp / 16) of the rows l / (Dp / 16) + k * RG,
// all its loads in flight together; the column sums add the lanes of one
// piece, the row distances the pieces of a row.
template <int DP>
__global__ void __launch_bounds__(256) chunk_bounds_kernel(const int8_t* __restrict__ X8,
                                                           const int32_t* __restrict__ pool,
                                                           const int32_t* __restrict__ cnt, int64_t nch,
                                                           int8_t* __restrict__ c8, float* __restrict__ cn,
                                                           float* __restrict__ cr)
{
    constexpr int PC = DP / 16;          // pieces per row
    constexpr int RG = 64 / PC;          // row groups per wave
    constexpr int RPT = kChunkRows / RG; // rows per lane
    static_assert((PC & (PC - 1)) == 0 && PC <= 16, "chunk shape");
    __shared__ int32_t cs[4][DP];
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int64_t g = static_cast<int64_t>(blockIdx.x) * 4 + w;
    if (g >= nch) return;
    const int q = lane % PC, rg = lane / PC;
    const int n = cnt[g];
    int32_t id[RPT];
#pragma unroll
    for (int k = 0; k < RPT; ++k) {
        const int r = rg + k * RG;
        id[k] = r < n ? pool[g * kChunkRows + r] : -1;
    }
    intx4 x[RPT];
#pragma unroll
    for (int k = 0; k < RPT; ++k)
        x[k] = id[k] >= 0 ? *reinterpret_cast<const intx4*>(X8 + static_cast<int64_t>(id[k]) * DP + 16 * q)
                          : intx4{0, 0, 0, 0};
    int sum[16];
#pragma unroll
    for (int b = 0; b < 16; ++b) {
        int sb = 0;
#pragma unroll
        for (int k = 0; k < RPT; ++k) sb += static_cast<int8_t>(x[k][b >> 2] >> (8 * (b & 3)));
        sum[b] = sb;
    }
    // the lanes of one piece (stride PC)
#pragma unroll
    for (int o = PC; o < 64; o <<= 1)
#pragma unroll
        for (int b = 0; b < 16; ++b) sum[b] += __shfl_xor(sum[b], o);
    int nsum = 0;
    if (lane < PC) {
        const float inv = 1.0f / static_cast<float>(n > 0 ? n : 1);
#pragma unroll
        for (int b = 0; b < 16; ++b) {
            const int c = n > 0 ? static_cast<int>(rintf(static_cast<float>(sum[b]) * inv)) : 0;
            cs[w][16 * q + b] = c;
            c8[g * DP + 16 * q + b] = static_cast<int8_t>(c);
            nsum += c * c;
        }
    }
    wave_sync();
    // each row's |p - c|^2: the PC lanes of a row (consecutive) add
    int v = 0;
#pragma unroll
    for (int k = 0; k < RPT; ++k) {
        int d = 0;
#pragma unroll
        for (int b = 0; b < 16; ++b) {
            const int e = static_cast<int>(static_cast<int8_t>(x[k][b >> 2] >> (8 * (b & 3)))) - cs[w][16 * q + b];
            d += e * e;
        }
#pragma unroll
        for (int o = 1; o < PC; o <<= 1) d += __shfl_xor(d, o);
        if (id[k] >= 0) v = max(v, d);
    }
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) {
        nsum += __shfl_xor(nsum, o);
        v = max(v, __shfl_xor(v, o));
    }
    if (lane == 0) {
        cn[g] = static_cast<float>(nsum);
        cr[g] = sqrtf(static_cast<float>(v)) * 1.000001f;
    }
}

void launch_chunk_bounds(const int8_t* X8, int Dp, const int32_t* pool, const int32_t* cnt, int64_t nch, int8_t* c8,
                         float* cn, float* cr, hipStream_t s)
{
    if (nch <= 0) return;
    const dim3 grid(static_cast<unsigned>((nch + 3) / 4));
    switch (Dp) {
    case 32: hipLaunchKernelGGL((chunk_bounds_kernel<32>), grid, dim3(256), 0, s, X8, pool, cnt, nch, c8, cn, cr); break;
    case 64: hipLaunchKernelGGL((chunk_bounds_kernel<64>), grid, dim3(256), 0, s, X8, pool, cnt, nch, c8, cn, cr); break;
    case 128: hipLaunchKernelGGL((chunk_bounds_kernel<128>), grid, dim3(256), 0, s, X8, pool, cnt, nch, c8, cn, cr); break;
    case 256: hipLaunchKernelGGL((chunk_bounds_kernel<256>), grid, dim3(256), 0, s, X8, pool, cnt, nch, c8, cn, cr); break;
    default: GT_REQUIRE(false, "chunk bounds: padded dimension " + std::to_string(Dp) + " not supported");
    }
    GT_HIP(hipGetLastError());
}

// ------------------------------------------------------------ host side

// Shapes the collect + select kernels take (the context's knn_collect
// option can keep the merging kernel for every list; same results)
bool knn_collect_supported(const KnnArgs& a)
{
    if (!(a.M > 4 && a.M <= 64 && a.out_pos == 0 && a.Dp % 32 == 0)) return false;
    if (a.Xq8 && a.Xp8) return a.Dp <= 256;
    return a.Xq && a.Xp && a.Dp <= 160;   // longer fp32 rows: the query fragment leaves too few registers
}

template <int METRIC>
static void launch_collect_f32_metric(const KnnArgs& a, dim3 grid, hipStream_t stream)
{
    switch (a.Dp) {
    case 32:  hipLaunchKernelGGL((knn_f32_collect_kernel<32, METRIC>), grid, dim3(256), 0, stream, a); break;
    case 64:  hipLaunchKernelGGL((knn_f32_collect_kernel<64, METRIC>), grid, dim3(256), 0, stream, a); break;
    case 96:  hipLaunchKernelGGL((knn_f32_collect_kernel<96, METRIC>), grid, dim3(256), 0, stream, a); break;
    case 128: hipLaunchKernelGGL((knn_f32_collect_kernel<128, METRIC>), grid, dim3(256), 0, stream, a); break;
    case 160: hipLaunchKernelGGL((knn_f32_collect_kernel<160, METRIC>), grid, dim3(256), 0, stream, a); break;
    default: GT_REQUIRE(false, "fp32 collect kernel: padded dimension " + std::to_string(a.Dp) + " not supported");
    }
}

template <int METRIC>
static void launch_collect_metric(const KnnArgs& a, dim3 grid, hipStream_t stream)
{
    switch (a.Dp) {
    case 32:  hipLaunchKernelGGL((knn_i8_collect_kernel<32, METRIC>), grid, dim3(256), 0, stream, a); break;
    case 64:  hipLaunchKernelGGL((knn_i8_collect_kernel<64, METRIC>), grid, dim3(256), 0, stream, a); break;
    case 96:  hipLaunchKernelGGL((knn_i8_collect_kernel<96, METRIC>), grid, dim3(256), 0, stream, a); break;
    case 128: hipLaunchKernelGGL((knn_i8_collect_kernel<128, METRIC>), grid, dim3(256), 0, stream, a); break;
    case 160: hipLaunchKernelGGL((knn_i8_collect_kernel<160, METRIC>), grid, dim3(256), 0, stream, a); break;
    case 192: hipLaunchKernelGGL((knn_i8_collect_kernel<192, METRIC>), grid, dim3(256), 0, stream, a); break;
    case 224: hipLaunchKernelGGL((knn_i8_collect_kernel<224, METRIC>), grid, dim3(256), 0, stream, a); break;
    case 256: hipLaunchKernelGGL((knn_i8_collect_kernel<256, METRIC>), grid, dim3(256), 0, stream, a); break;
    default: GT_REQUIRE(false, "collect kernel: padded dimension " + std::to_string(a.Dp) + " not supported");
    }
}

// Every output row in [0, rows) must be the output row of exactly one query
// of the launch (cand_cnt is read for all of them); a.cand holds
// (rows + kQueriesPerWave) * kCollectCap keys.
void launch_knn_collect_select(const KnnArgs& a, int64_t rows, hipStream_t stream)
{
    GT_REQUIRE(knn_collect_supported(a), "collect launch: int8 rows (Dp <= 256) or fp32 rows (Dp <= 160), 4 < M <= 64");
    GT_REQUIRE(a.cand && a.cand_cnt && a.out_ids && a.out_d && a.p_rows, "collect launch: buffers missing");
    GT_REQUIRE(a.n_items % 8 == 0, "work list must be padded to a multiple of 8");
    if (a.n_items > 0) {
        const dim3 grid(static_cast<unsigned>(a.n_items));
        const bool i8 = a.Xq8 && a.Xp8;
        if (i8 && a.metric == 0) launch_collect_metric<0>(a, grid, stream);
        else if (i8) launch_collect_metric<1>(a, grid, stream);
        else if (a.metric == 0) launch_collect_f32_metric<0>(a, grid, stream);
        else launch_collect_f32_metric<1>(a, grid, stream);
        GT_HIP(hipGetLastError());
    }
    if (rows <= 0) return;
    const bool merge = a.run_ids != nullptr;
    GT_REQUIRE(!merge || (a.run_d && a.seed_d && a.seed_ld == a.M), "collect merge: running table missing");
    const dim3 sgrid(static_cast<unsigned>(ceil_div(rows, kQueriesPerBlock)));
    const dim3 mgrid(static_cast<unsigned>(ceil_div(rows, int64_t(64) * kWaves)));
    if (merge && a.Xq8 && a.Xp8) {
        // int8 rows: duplicates dropped and the rows with at most M fresh keys
        // merged; the others selected from the list and merged after
        GT_REQUIRE(a.hl_rows && a.hl_count, "collect merge: row list missing");
        GT_HIP(hipMemsetAsync(a.hl_count, 0, sizeof(uint32_t), stream));
        hipLaunchKernelGGL((knn_merge_fresh_kernel<kFreshRing>), mgrid, dim3(256), 0, stream, a.cand, a.cand_cnt,
                           rows, a.M, a.run_ids, a.run_d, a.hl_rows, a.hl_count, a.stats);
        GT_HIP(hipGetLastError());
        if (a.M <= 32)
            hipLaunchKernelGGL((knn_select_kernel<16, true>), sgrid, dim3(256), 0, stream, a.cand, a.cand_cnt, rows,
                               a.M, -1, a.hl_rows, a.hl_count, a.out_ids, a.out_d);
        else
            hipLaunchKernelGGL((knn_select_kernel<32, true>), sgrid, dim3(256), 0, stream, a.cand, a.cand_cnt, rows,
                               a.M, -1, a.hl_rows, a.hl_count, a.out_ids, a.out_d);
        GT_HIP(hipGetLastError());
        constexpr int kListRpw = 4;   // few rows per wave: the list is short and its rows heavy
        hipLaunchKernelGGL(knn_merge_run_kernel, dim3(static_cast<unsigned>(ceil_div(rows, int64_t(kListRpw) * kWaves))),
                           dim3(256), 0, stream, a.cand, a.cand_cnt, rows, a.M, kListRpw, 0, a.hl_rows, a.hl_count,
                           a.out_ids, a.out_d, a.run_ids, a.run_d);
        GT_HIP(hipGetLastError());
        return;
    }
    // fp32 rows merged: rows of at most kRankMax keys ranked in the merge,
    // the others selected first
    constexpr int kRankMax = 8;
    const int skip_le = merge ? kRankMax : -1;
    if (a.M <= 32)
        hipLaunchKernelGGL((knn_select_kernel<16, false>), sgrid, dim3(256), 0, stream, a.cand, a.cand_cnt, rows,
                           a.M, skip_le, nullptr, nullptr, a.out_ids, a.out_d);
    else
        hipLaunchKernelGGL((knn_select_kernel<32, false>), sgrid, dim3(256), 0, stream, a.cand, a.cand_cnt, rows,
                           a.M, skip_le, nullptr, nullptr, a.out_ids, a.out_d);
    GT_HIP(hipGetLastError());
    if (merge) {
        hipLaunchKernelGGL(knn_merge_run_kernel, mgrid, dim3(256), 0, stream, a.cand, a.cand_cnt, rows, a.M, 64,
                           kRankMax, nullptr, nullptr, a.out_ids, a.out_d, a.run_ids, a.run_d);
        GT_HIP(hipGetLastError());
    }
}

}  // namespace gtann
