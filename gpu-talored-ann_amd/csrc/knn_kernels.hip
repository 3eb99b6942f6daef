// knn_kernels.hip -- per-bucket brute-force kNN for gfx950.
//
// One workgroup (4 waves) scans a contiguous slice of a pool list for a tile
// of 128 query rows.  The |x|^2 - 2x.y contraction runs on the fp32 matrix
// cores (v_mfma_f32_32x32x2_f32) with the pool tile staged through LDS and
// each wave's 32 query rows held in registers; the 32x32 distance block is
// filtered in registers against each query's current M-th key and only the
// survivors are appended to a per-query LDS buffer, which is merged into the
// query's sorted list when it fills.  The (queries x pool) distance matrix
// never reaches HBM.
//
// Semantics follow the reference's top-M (src/bucket.cu:4101-4265): self is
// excluded, padding is (-1, +inf), distance reported = |q|^2 + |p|^2 - 2 q.p.
// Ties are ordered by id (total order (key, id)), so the kept set and its
// order are unique.
#include "knn_device.hpp"

#include <algorithm>
#include <cfloat>
#include <climits>
#include <cmath>

namespace gtann {


constexpr int kCB = 32;      // candidate-buffer slots per query (>= 32 = one tile's worth per query)
constexpr int kMaxM = 128;   // longest list the kernel keeps

__device__ __forceinline__ bool key_less(float da, int32_t ia, float db, int32_t ib)
{
    return da < db || (da == db && ia < ib);
}

// number of entries of the sorted (d, i) array [0, n) that are < (kd, ki)
__device__ __forceinline__ int lower_bound_lds(const float* ad, const int32_t* ai, int n, float kd, int32_t ki)
{
    int lo = 0, hi = n;
    while (lo < hi) {
        const int mid = (lo + hi) >> 1;
        if (key_less(ad[mid], ai[mid], kd, ki)) lo = mid + 1;
        else hi = mid;
    }
    return lo;
}

// Per-block candidate buffers and merge staging, shared by both kernels.
struct KnnLists {
    // packed (key, id) of candidates awaiting a merge (never the query
    // itself); slot kCB takes the writes of rows that did not pass (branch-free
    // appends) and is never read
    uint64_t buf[kQueriesPerBlock][kCB + 2];
    uint64_t lst[kWaves][kMaxM];          // the merging query's list, packed
};

template <int DP>
struct KnnSmemTiles {
    float tile[2][kPoolTile][DP + 4];   // +4 floats: rows land on distinct bank groups
    float tnorm[3][kPoolTile];          // |p|^2 (L2) or 0 (IP); +inf past the slice end
    int32_t trow[3][kPoolTile];         // pool row id, -1 past the slice end
    int32_t sid[2][kPoolTile];          // the next tile's pool row ids, for every thread's row requests
};

template <int DP, bool LISTS = true>
struct KnnSmem : KnnSmemTiles<DP> {
    KnnLists L;
};

template <int DP>
struct KnnSmem<DP, false> : KnnSmemTiles<DP> {};

// Per-lane view of one query's state.  Lanes j and j+32 of a wave hold the
// same query (both halves of the MFMA's k split) and keep identical copies.
struct QueryState {
    float thr;     // keep a candidate iff key <= thr (finite: never admits a +inf key)
    float seed;    // cap from the caller (previous round's M-th), FLT_MAX if none
    int32_t cnt;   // entries in the LDS buffer
    int32_t nL;    // entries in the sorted list (stored in the output row)
    int32_t self;  // id that must not be kept (the query itself), -2 if none
    int64_t orow;  // output row
};


// A list row is only ever stored and loaded by the one wave that owns its
// query, on one CU: workgroup-scope loads see those stores once they have
// completed (the vmcnt(0) waits above), and being atomic they are never
// folded with an earlier load of the same row by the compiler.
__device__ __forceinline__ float load_list_d(const float* p)
{
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}
__device__ __forceinline__ int32_t load_list_i(const int32_t* p)
{
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}


// Merges the buffer of query q (0..31 of this wave) into its sorted list
// (output row) and recomputes its threshold.  A buffer entry goes to its rank
// among the buffer plus the number of list entries below it; a list entry to
// its index plus the number of buffer entries below it.  The buffer ranks
// come from counting (split between the two half-waves, lanes l and l + 32
// both holding buffer entry l, over 128-bit LDS broadcast reads); the buffer
// then sits in LDS in rank order, each list entry finds its count by a lower
// bound in it, and the list entries below the buffer entry of rank r are
// those whose lower bound is at most r: a prefix sum (DPP) over a histogram
// of the lower bounds.  Keys are distinct, so no count is ambiguous.  The
// list loads are issued first and land while the buffer is ranked.  Called by
// all 64 lanes.
__device__ void wave_merge(KnnLists& sm, const KnnArgs& a, int w, int lane, int q, QueryState& st)
{
    // query q's state, uniform across the wave (scalar registers)
    const int nL = __builtin_amdgcn_readlane(st.nL, q);
    const int64_t orow = static_cast<int64_t>(
        (static_cast<uint64_t>(static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(st.orow >> 32), q))) << 32) |
        static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(st.orow), q)));
    const int M = a.M;
    const int h = lane >> 5;
    uint64_t* B = sm.buf[w * kQueriesPerWave + q];
    uint64_t* L = sm.lst[w];

    float ld0 = 0.f, ld1 = 0.f;
    int32_t li0 = 0, li1 = 0;
    if (lane < nL) {
        ld0 = load_list_d(a.out_d + orow * M + lane);
        li0 = load_list_i(a.out_ids + orow * M + lane);
    }
    if (lane + 64 < nL) {
        ld1 = load_list_d(a.out_d + orow * M + lane + 64);
        li1 = load_list_i(a.out_ids + orow * M + lane + 64);
    }

    // buffer slots past nB hold kNoKey (never below a key)
    const int bl = lane & 31;
    const uint64_t bk = B[bl];
    auto key_at = [](const uint4& x, int odd) -> uint64_t {
        return odd ? (static_cast<uint64_t>(x.w) << 32) | x.z : (static_cast<uint64_t>(x.y) << 32) | x.x;
    };
    // rank of buffer entry bl among the buffer: half h counts entries [16h, 16h + 16)
    int rb = 0;
    {
        const uint4* B4 = reinterpret_cast<const uint4*>(B + 16 * h);
#pragma unroll 4
        for (int e = 0; e < 8; ++e) {
            const uint4 x = B4[e];
#pragma unroll
            for (int o = 0; o < 2; ++o) rb += key_at(x, o) < bk ? 1 : 0;
        }
    }
    rb += __shfl_xor(rb, 32);

    // the buffer in key order through LDS (slots past the valid entries
    // hold kNoKey): S[rank] = key
    const bool bvalid = h == 0 && bk != kNoKey;
    uint64_t* S = L;
    if (h == 0) S[bl] = kNoKey;
    if (bvalid) S[rb] = bk;
    if (h == 0) B[bl] = kNoKey;   // the buffer starts over empty
    wave_sync();

    // buffer entries below list entries lane, lane + 64: lower bounds in S,
    // over S[0, 31) in five halvings, then S[31]
    const uint64_t lk0 = lane < nL ? pack_key(ld0, li0) : kNoKey;
    const uint64_t lk1 = lane + 64 < nL ? pack_key(ld1, li1) : kNoKey;
    int cl0 = 0, cl1 = 0;
#pragma unroll
    for (int step = 16; step > 0; step >>= 1) {
        if (S[cl0 + step - 1] < lk0) cl0 += step;
        if (nL > 64 && S[cl1 + step - 1] < lk1) cl1 += step;
    }
    cl0 += S[cl0] < lk0 ? 1 : 0;
    if (nL > 64) cl1 += S[cl1] < lk1 ? 1 : 0;

    // list entries below the buffer entry of rank r: those with cl <= r (the
    // list is sorted and keys are distinct), a prefix sum over r of the
    // histogram of cl, kept in LDS after S
    int* H = reinterpret_cast<int*>(L + 32);   // counters 0..32
    if (lane <= 32) H[lane] = 0;
    wave_sync();
    if (lane < nL) atomicAdd(&H[cl0], 1);
    if (lane + 64 < nL) atomicAdd(&H[cl1], 1);
    wave_sync();
    const int below = wave_incl_scan(lane <= 32 ? H[lane] : 0);
    const int nlb = __shfl(below, rb);

    const int nBv = static_cast<int>(__popcll(__ballot(bvalid)));
    const int total = nL + nBv;
    bool last = false;   // this lane wrote position M-1
    float dlast = 0.f;
    if (bvalid) {
        const int pos = rb + nlb;
        if (pos < M) {
            const float d = o2f(static_cast<uint32_t>(bk >> 32));
            a.out_d[orow * M + pos] = d;
            a.out_ids[orow * M + pos] = static_cast<int32_t>(static_cast<uint32_t>(bk));
            if (pos == M - 1) { last = true; dlast = d; }
        }
    }
    if (lane < nL) {
        const int pos = lane + cl0;
        if (pos < M) {
            a.out_d[orow * M + pos] = ld0;
            a.out_ids[orow * M + pos] = li0;
            if (pos == M - 1) { last = true; dlast = ld0; }
        }
    }
    if (lane + 64 < nL) {
        const int pos = lane + 64 + cl1;
        if (pos < M) {
            a.out_d[orow * M + pos] = ld1;
            a.out_ids[orow * M + pos] = li1;
            if (pos == M - 1) { last = true; dlast = ld1; }
        }
    }
    const uint64_t lastmask = __ballot(last);
    float mth = FLT_MAX;
    if (lastmask) {
        const int src = static_cast<int>(__ffsll(static_cast<unsigned long long>(lastmask))) - 1;
        mth = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(dlast), src));
    }
    const int newn = total < M ? total : M;
    if ((lane & 31) == q) {
        st.cnt = 0;
        st.nL = newn;
        st.thr = (newn == M) ? fminf(st.seed, mth) : st.seed;
    }
}

// Lists of at most kSmallM entries (top-2 assignment, Lloyd, narrow probe
// tables) are merged for every query of the wave at once, one lane per
// query (lanes 0..31): the list goes into registers and each buffer entry is
// inserted by one compare-exchange pass.  A wave-wide merge per query would
// cost as much as the whole scan of such a short pool.
constexpr int kSmallM = 4;

__device__ void small_merge_all(KnnLists& sm, const KnnArgs& a, int w, int lane, uint64_t mask, QueryState& st)
{
    const int M = a.M;
    if (lane < 32 && ((mask >> lane) & 1ull)) {
        const int64_t row = st.orow * M;
        uint64_t k[kSmallM];
#pragma unroll
        for (int i = 0; i < kSmallM; ++i)
            k[i] = i < st.nL ? pack_key(load_list_d(a.out_d + row + i), load_list_i(a.out_ids + row + i)) : kNoKey;
        uint64_t* B = sm.buf[w * kQueriesPerWave + lane];
        for (int e = 0; e < st.cnt; ++e) {
            uint64_t x = B[e];
            B[e] = kNoKey;   // the buffer starts over empty
#pragma unroll
            for (int i = 0; i < kSmallM; ++i) {
                const bool lt = x < k[i];
                const uint64_t lo = lt ? x : k[i];
                x = lt ? k[i] : x;
                k[i] = lo;
            }
        }
        const int newn = min(st.nL + st.cnt, M);
        float mth = 0.f;
#pragma unroll
        for (int i = 0; i < kSmallM; ++i) {
            if (i < newn) {
                const float d = o2f(static_cast<uint32_t>(k[i] >> 32));
                a.out_d[row + i] = d;
                a.out_ids[row + i] = static_cast<int32_t>(static_cast<uint32_t>(k[i]));
                if (i == M - 1) mth = d;
            }
        }
        st.cnt = 0;
        st.nL = newn;
        st.thr = newn == M ? fminf(st.seed, mth) : st.seed;
    }
    // the second half-wave holds the same queries' state
    st.cnt = __shfl(st.cnt, lane & 31);
    st.nL = __shfl(st.nL, lane & 31);
    st.thr = __shfl(st.thr, lane & 31);
    wave_sync();
}

// Merges the buffers of the queries in `mask` (bit q = query q of the wave).
// SMALL: the launch may have lists of at most kSmallM entries (the int8
// kernel never does: its registers stay below the three-wave limit).
template <bool SMALL>
__device__ __forceinline__ void merge_queries(KnnLists& sm, const KnnArgs& a, int w, int lane, uint64_t mask,
                                              QueryState& st)
{
    if (SMALL && a.M <= kSmallM) {
        small_merge_all(sm, a, w, lane, mask, st);
        return;
    }
    while (mask) {
        const int q = __ffsll(static_cast<unsigned long long>(mask)) - 1;
        mask &= mask - 1;
        wave_merge(sm, a, w, lane, q, st);
    }
}

// Lists of at most kSmallM entries in registers: every lane keeps the best
// keys among the pool rows it holds (its half of each tile); the two halves
// of a query are merged once, at the end.  No LDS buffer, no merges.
struct SmallList {
    uint64_t k[kSmallM];   // ascending, kNoKey = empty
    float kth;             // a candidate is kept iff its distance <= kth
};

__device__ __forceinline__ void small_insert(SmallList& L, uint64_t x)
{
#pragma unroll
    for (int i = 0; i < kSmallM; ++i) {
        const bool lt = x < L.k[i];
        const uint64_t lo = lt ? x : L.k[i];
        x = lt ? L.k[i] : x;
        L.k[i] = lo;
    }
}

__device__ __forceinline__ void small_update_kth(SmallList& L, int M, float seed)
{
    const uint64_t km = M <= 1 ? L.k[0] : M == 2 ? L.k[1] : M == 3 ? L.k[2] : L.k[3];
    L.kth = km == kNoKey ? seed : fminf(seed, o2f(static_cast<uint32_t>(km >> 32)));
}

// One finished 32x32 tile into the lane's register list.
template <int METRIC, typename Acc>
__device__ __forceinline__ void small_tile(const KnnArgs& a, const Acc& acc, const float* tn, const int32_t* tr,
                                           int tbase, int h, bool qvalid, float qn, const QueryState& st,
                                           SmallList& L)
{
    float dv[16];
#pragma unroll
    for (int g = 0; g < 4; ++g) {
        const float4 pn = *reinterpret_cast<const float4*>(tn + 8 * g + 4 * h);
        const float n4[4] = {pn.x, pn.y, pn.z, pn.w};
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const float dot = static_cast<float>(acc[4 * g + e]);
            dv[4 * g + e] = METRIC == 0 ? fmaf(-2.f, dot, n4[e] + qn) : fmaf(-1.f, dot, n4[e]);
        }
    }
    uint32_t pass = 0;
#pragma unroll
    for (int r = 0; r < 16; ++r) pass |= static_cast<uint32_t>(qvalid && dv[r] <= L.kth) << r;
    if (!__ballot(pass != 0u)) return;
    int32_t idv[16];
#pragma unroll
    for (int g = 0; g < 4; ++g) {
        const int4 pi = *reinterpret_cast<const int4*>(tr + 8 * g + 4 * h);
        const int32_t i4[4] = {pi.x, pi.y, pi.z, pi.w};
#pragma unroll
        for (int e = 0; e < 4; ++e) idv[4 * g + e] = a.out_pos ? tbase + 8 * g + 4 * h + e : i4[e];
    }
#pragma unroll
    for (int r = 0; r < 16; ++r) pass &= ~(static_cast<uint32_t>(idv[r] == st.self) << r);
#pragma unroll
    for (int r = 0; r < 16; ++r)
        if (__ballot((pass >> r) & 1u))
            if ((pass >> r) & 1u) small_insert(L, pack_key(dv[r], idv[r]));
    small_update_kth(L, a.M, st.seed);
    // the query's two half-lists each hold M keys at or below their own
    // M-th distance, so a candidate above the smaller of the two can never
    // enter the merged top M: both halves filter with it
    L.kth = fminf(L.kth, __shfl_xor(L.kth, 32));
}

// The second half-wave's keys join the first half's list, which lane j
// writes to output row orow (padding -1 / +inf).
__device__ __forceinline__ void small_finish(const KnnArgs& a, SmallList& L, int j, int h, bool qvalid, int64_t orow)
{
    uint64_t other[kSmallM];
#pragma unroll
    for (int i = 0; i < kSmallM; ++i) other[i] = __shfl(L.k[i], j + 32);
    if (qvalid && h == 0) {
#pragma unroll
        for (int i = 0; i < kSmallM; ++i) small_insert(L, other[i]);
        for (int p = 0; p < a.M; ++p) {
            const uint64_t kp = p == 0 ? L.k[0] : p == 1 ? L.k[1] : p == 2 ? L.k[2] : L.k[3];
            a.out_ids[orow * a.M + p] = kp == kNoKey ? -1 : static_cast<int32_t>(static_cast<uint32_t>(kp));
            a.out_d[orow * a.M + p] = kp == kNoKey ? INFINITY : o2f(static_cast<uint32_t>(kp >> 32));
        }
    }
}

// Filter + append of one finished 32x32 tile whose pool rows have norms
// tn[0..32) and ids tr[0..32) (tbase = pool-list position of row 0), the slow
// path taken only when some lane of the wave has a candidate <= its threshold.
template <int METRIC, bool SMALL>
__device__ __forceinline__ void tile_append(KnnLists& sm, const KnnArgs& a, const floatx16& acc, const float* tn,
                                            const int32_t* tr, int tbase, int w, int lane, int h, int qlocal,
                                            bool qvalid, float qn, QueryState& st)
{
    // rows 8g + 4h + e of the tile, e = 0..3: norms and ids as 128-bit reads
    float dv[16];
    int32_t idv[16];
#pragma unroll
    for (int g = 0; g < 4; ++g) {
        const float4 pn = *reinterpret_cast<const float4*>(tn + 8 * g + 4 * h);
        const int4 pi = *reinterpret_cast<const int4*>(tr + 8 * g + 4 * h);
        const float n4[4] = {pn.x, pn.y, pn.z, pn.w};
        const int32_t i4[4] = {pi.x, pi.y, pi.z, pi.w};
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int r = 4 * g + e;
            dv[r] = METRIC == 0 ? fmaf(-2.f, acc[r], n4[e] + qn) : fmaf(-1.f, acc[r], n4[e]);
            idv[r] = a.out_pos ? tbase + 8 * g + 4 * h + e : i4[e];
        }
    }
    uint32_t keep = 0;   // rows that may enter the list: not the query itself
#pragma unroll
    for (int r = 0; r < 16; ++r) keep |= static_cast<uint32_t>(idv[r] != st.self) << r;
    uint32_t pass = 0;
#pragma unroll
    for (int r = 0; r < 16; ++r) pass |= static_cast<uint32_t>(dv[r] <= st.thr) << r;
    pass &= keep;
    int np_ = __popc(pass);
    int np_o = __shfl_xor(np_, 32);
    const bool need = qvalid && (st.cnt + np_ + np_o > kCB);
    uint64_t needmask = __ballot(need) & 0xffffffffull;
    if (needmask) {
        merge_queries<SMALL>(sm, a, w, lane, needmask, st);
        pass = 0;
#pragma unroll
        for (int r = 0; r < 16; ++r) pass |= static_cast<uint32_t>(dv[r] <= st.thr) << r;
        pass &= keep;
        np_ = __popc(pass);
        np_o = __shfl_xor(np_, 32);
    }
    if (qvalid) {
        // half 0 fills slots [cnt, cnt + np_), half 1 the next np_o; rows that
        // did not pass go to the spare slot kCB
        const int base = st.cnt + (h ? np_o : 0);
        uint64_t* row = sm.buf[qlocal];
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int slot = ((pass >> r) & 1u) ? base + __popc(pass & ((1u << r) - 1u)) : kCB;
            row[slot] = pack_key(dv[r], idv[r]);
        }
        st.cnt += np_ + np_o;
    }
}

// SMALL: lists of at most kSmallM entries, kept in registers (SmallList).
template <int DP, int METRIC, bool SMALL>
__global__ void __launch_bounds__(256, 2) knn_fused_kernel(KnnArgs a)
{
    constexpr int DH = DP / 2;                    // k-steps of 2 dims (one per half wave)
    constexpr int F4_ROW = DP / 4;
    constexpr int F4_THREAD = kPoolTile * F4_ROW / 256;
    static_assert(DP % 32 == 0, "row stride must be a multiple of 32 floats");
    __shared__ KnnSmem<DP, !SMALL> sm;

    // Work items are laid out XCD-major by the host: the hardware deals
    // consecutive workgroups round-robin over the 8 XCDs, so XCD x runs items
    // [x*per, (x+1)*per) in order (same bucket => same pool rows => shared L2).
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

    QueryState st;
    st.seed = FLT_MAX;
    // the seed is read from the output row (the query row unless the item has an out_base)
    const int64_t orow_seed = it.out_base >= 0 ? it.out_base + qlocal : static_cast<int64_t>(qrow);
    if (qvalid && a.seed_d) st.seed = fminf(a.seed_d[orow_seed * a.seed_ld + a.seed_ld - 1], FLT_MAX);
    st.thr = qvalid ? st.seed : -INFINITY;
    st.cnt = 0;
    st.nL = 0;
    st.self = a.exclude_self ? qrow : -2;
    st.orow = it.out_base >= 0 ? it.out_base + qlocal : static_cast<int64_t>(qrow);
    SmallList SL;
    if constexpr (SMALL) {
#pragma unroll
        for (int i = 0; i < kSmallM; ++i) SL.k[i] = kNoKey;
        SL.kth = st.thr;
    } else {
        // this wave's 32 buffer rows start empty: every slot holds kNoKey
        for (int e = lane; e < kQueriesPerWave * kCB; e += 64) sm.L.buf[w * kQueriesPerWave + e / kCB][e % kCB] = kNoKey;
    }

    // query fragment: dims [h*DH, h*DH + DH) of query row qrow
    float qf[DH];
    {
        const float4* src = reinterpret_cast<const float4*>(a.Xq + static_cast<int64_t>(qrow) * DP + h * DH);
#pragma unroll
        for (int s = 0; s < DH / 4; ++s) {
            const float4 v = qvalid ? src[s] : make_float4(0.f, 0.f, 0.f, 0.f);
            qf[4 * s + 0] = v.x; qf[4 * s + 1] = v.y; qf[4 * s + 2] = v.z; qf[4 * s + 3] = v.w;
        }
    }

    const int pcount = it.p_count;
    const int ntiles = (pcount + kPoolTile - 1) / kPoolTile;
    auto pool_row = [&](int p) -> int32_t {
        if (p >= pcount) return -1;
        p += it.p_rot;
        if (p >= pcount) p -= pcount;
        const int64_t pl = it.p_begin + p;
        return a.p_rows ? a.p_rows[pl] : static_cast<int32_t>(pl);
    };
    auto row_norm = [&](int32_t row) -> float {
        if (row < 0) return INFINITY;
        return METRIC == 0 ? a.np[row] : 0.f;
    };

    // Pool tiles flow through three stages: ids (two tiles ahead, fetched by
    // the threads < 32, one per row, and handed to every thread through LDS)
    // -> row data in registers (one tile ahead) -> LDS.  Thread tid loads
    // float4 c4_u of tile row r_u; threads < 32 also carry the id and norm of
    // row tid.
    float4 pre[F4_THREAD];
    int32_t rid_next = -1;   // id of row tid two tiles ahead (tid < 32)
    auto load_rows = [&](const int32_t* ids) {
#pragma unroll
        for (int u = 0; u < F4_THREAD; ++u) {
            const int e = tid + 256 * u;
            const int32_t id = ids[e / F4_ROW];
            pre[u] = id >= 0 ? reinterpret_cast<const float4*>(a.Xp + static_cast<int64_t>(id) * DP)[e % F4_ROW]
                             : make_float4(0.f, 0.f, 0.f, 0.f);
        }
    };
    auto store_rows = [&](int buf) {
#pragma unroll
        for (int u = 0; u < F4_THREAD; ++u) {
            const int e = tid + 256 * u;
            *reinterpret_cast<float4*>(&sm.tile[buf][e / F4_ROW][4 * (e % F4_ROW)]) = pre[u];
        }
    };

    int32_t rid_cur = -1;
    float rn_cur = 0.f;
    if (tid < kPoolTile) {
        sm.tnorm[2][tid] = INFINITY; sm.trow[2][tid] = -1;
        rid_cur = pool_row(tid);
        sm.sid[0][tid] = rid_cur;
        rn_cur = row_norm(rid_cur);
        rid_next = pool_row(kPoolTile + tid);
    }
    __syncthreads();
    load_rows(sm.sid[0]);
    store_rows(0);
    if (tid < kPoolTile) { sm.trow[0][tid] = rid_cur; sm.tnorm[0][tid] = rn_cur; sm.sid[1][tid] = rid_next; }
    __syncthreads();

    floatx16 acc_prev;
#pragma unroll
    for (int r = 0; r < 16; ++r) acc_prev[r] = 0.f;

    for (int t = 0; t < ntiles; ++t) {
        const int buf = t & 1;
        wait_vmem();   // ids of the tile after next, and any list rows stored by merges
        // next tile: rows (their ids in LDS since the previous tile) and norms
        load_rows(sm.sid[(t + 1) & 1]);
        if (tid < kPoolTile) {
            rid_cur = rid_next;
            rn_cur = row_norm(rid_cur);
            rid_next = pool_row((t + 2) * kPoolTile + tid);   // tile after next: ids
        }

        // D[i][j] = sum_k pool[i][k] * query[j][k]; lane supplies A[i=lane%32][k=lane/32]
        // (pool row j, dim h*DH+s) and B[k=lane/32][j=lane%32] (query j, same dim).
        floatx16 acc;
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[r] = 0.f;
        const float* arow = &sm.tile[buf][j][h * DH];
#pragma unroll
        for (int s = 0; s < DH / 4; ++s) {
            const float4 av = *reinterpret_cast<const float4*>(arow + 4 * s);
            acc = __builtin_amdgcn_mfma_f32_32x32x2f32(av.x, qf[4 * s + 0], acc, 0, 0, 0);
            acc = __builtin_amdgcn_mfma_f32_32x32x2f32(av.y, qf[4 * s + 1], acc, 0, 0, 0);
            acc = __builtin_amdgcn_mfma_f32_32x32x2f32(av.z, qf[4 * s + 2], acc, 0, 0, 0);
            acc = __builtin_amdgcn_mfma_f32_32x32x2f32(av.w, qf[4 * s + 3], acc, 0, 0, 0);
        }

        // Fast filter of the previous tile (t-1), independent of the MFMA
        // chain above: min key per lane.  acc_prev[r] is D[i][j] with
        // i = 8*(r/4) + 4*h + r%4.  Rows past the slice have +inf norm.
        const int pb3 = (t + 2) % 3;   // (t-1) mod 3
        if constexpr (SMALL) {
            if (t > 0)
                small_tile<METRIC>(a, acc_prev, sm.tnorm[pb3], sm.trow[pb3], (t - 1) * kPoolTile, h, qvalid, qn, st,
                                   SL);
        } else {
            float mkey = INFINITY;
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                const float4 pn = *reinterpret_cast<const float4*>(&sm.tnorm[pb3][8 * g + 4 * h]);
                const float n4[4] = {pn.x, pn.y, pn.z, pn.w};
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const float d = METRIC == 0 ? fmaf(-2.f, acc_prev[4 * g + e], n4[e] + qn)
                                                : fmaf(-1.f, acc_prev[4 * g + e], n4[e]);
                    mkey = fminf(mkey, d);
                }
            }
            if (t > 0 && __ballot(mkey <= st.thr))
                tile_append<METRIC, true>(sm.L, a, acc_prev, sm.tnorm[pb3], sm.trow[pb3], (t - 1) * kPoolTile, w,
                                           lane, h, qlocal, qvalid, qn, st);
        }

        store_rows(buf ^ 1);
        if (tid < kPoolTile) {
            sm.trow[(t + 1) % 3][tid] = rid_cur;
            sm.tnorm[(t + 1) % 3][tid] = rn_cur;
            sm.sid[t & 1][tid] = rid_next;   // tile t + 2's ids
        }
        __syncthreads();
        acc_prev = acc;
    }
    if constexpr (SMALL) {
        if (ntiles > 0) {
            wait_vmem();
            const int pb3 = (ntiles - 1) % 3;
            small_tile<METRIC>(a, acc_prev, sm.tnorm[pb3], sm.trow[pb3], (ntiles - 1) * kPoolTile, h, qvalid, qn, st,
                               SL);
        }
        small_finish(a, SL, j, h, qvalid, st.orow);
    } else {
        if (ntiles > 0) {
            wait_vmem();   // list rows stored by the last iteration's merges
            const int pb3 = (ntiles - 1) % 3;
            float mkey = INFINITY;
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int i = 8 * (r >> 2) + 4 * h + (r & 3);
                const float pn = sm.tnorm[pb3][i];
                mkey = fminf(mkey, METRIC == 0 ? fmaf(-2.f, acc_prev[r], pn + qn) : fmaf(-1.f, acc_prev[r], pn));
            }
            if (__ballot(mkey <= st.thr))
                tile_append<METRIC, true>(sm.L, a, acc_prev, sm.tnorm[pb3], sm.trow[pb3], (ntiles - 1) * kPoolTile, w,
                                           lane, h, qlocal, qvalid, qn, st);
        }

        // flush the remaining buffers
        wait_vmem();
        merge_queries<true>(sm.L, a, w, lane, __ballot(qvalid && st.cnt > 0) & 0xffffffffull, st);
        if (qvalid) {
            for (int p = st.nL + h; p < a.M; p += 2) {
                a.out_ids[st.orow * a.M + p] = -1;
                a.out_d[st.orow * a.M + p] = INFINITY;
            }
        }
    }
}

// ------------------------------------------------------------ int8 rows
//
// Integer-typed inputs (int8, or uint8 shifted by -128) run on the int8
// matrix cores: v_mfma_i32_32x32x32_i8 contracts 32 dimensions per step with
// exact int32 sums, so a 32x32 tile of D = 128 is 4 MFMAs instead of 64.
// Each lane holds its query's bytes [32s + 16h, 32s + 16h + 16) for every
// step s (the pool rows in LDS are read with the same split), so the two
// half-waves cover the row between them.  Keys are exact: |p|^2 + |q|^2 -
// 2 p.q < 2^24.  Filtering, appends and merges are the fp32 kernel's.

// Pool rows per stage (one barrier, one load round trip): with register
// short lists a 32x32 tile is a few MFMAs and no LDS list work, too short to
// hide a load latency, so those launches stage 4 tiles (2 for long rows).
template <int DP, bool SMALL>
struct I8Stage {
    static constexpr int SUB = SMALL ? (DP <= 128 ? 4 : 2) : 1;
    static constexpr int ROWS = kPoolTile * SUB;
};

template <int DP, int ROWS>
struct KnnSmemI8Tiles {
    int8_t tile[2][ROWS][DP + 16];   // +16 bytes: rows land on distinct bank groups
    float tnorm[3][ROWS];
    int32_t trow[3][ROWS];
    int32_t thalf[3][ROWS];          // accumulator start: -floor(|p|^2 / 2) (L2), 0 (IP), kHalfPast past the end
    int32_t sid[2][ROWS];            // the next stage's pool row ids (-1 past the end), for every thread's row requests
};



template <int DP, bool LISTS>
struct KnnSmemI8 : KnnSmemI8Tiles<DP, I8Stage<DP, !LISTS>::ROWS> {
    KnnLists L;
};

template <int DP>
struct KnnSmemI8<DP, false> : KnnSmemI8Tiles<DP, I8Stage<DP, true>::ROWS> {};


// One finished 32x32 tile of an int8 list launch: acc holds v = dot -
// floor(|p|^2 / 2) (L2) or dot (IP) for pool rows with norms tn, ids tr and
// accumulator starts th.  Tiles with no v at the query's pass floor lo are
// dropped; the others go through tile_append with the exact dot products,
// after which lo follows the query's (possibly lowered) threshold.
template <int METRIC>
__device__ __forceinline__ void i8_filter_tile(KnnLists& L, const KnnArgs& a, const intx16& acc, const float* tn,
                                               const int32_t* tr, const int32_t* th, int tbase, int w, int lane, int h,
                                               int qlocal, bool qvalid, float qn, QueryState& st, int32_t& lo)
{
    int32_t vmax = INT_MIN;
#pragma unroll
    for (int r = 0; r < 16; r += 2) vmax = max(vmax, max(acc[r], acc[r + 1]));
    if (__ballot(vmax >= lo)) {
        floatx16 dot;
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            const int4 hv = *reinterpret_cast<const int4*>(th + 8 * g + 4 * h);
            const int32_t h4[4] = {hv.x, hv.y, hv.z, hv.w};
#pragma unroll
            for (int e = 0; e < 4; ++e) dot[4 * g + e] = static_cast<float>(acc[4 * g + e] - h4[e]);
        }
        tile_append<METRIC, false>(L, a, dot, tn, tr, tbase, w, lane, h, qlocal, qvalid, qn, st);
        lo = i8_pass_floor<METRIC>(st.thr, qn);
    }
}

// One finished 32x32 tile of the resident short-list kernel, whose
// accumulators started at -floor(|p|^2 / 2) (L2) or 0 (IP) (th): a tile none
// of whose v reach the pass floor lo of the list's bound holds no row that
// small_tile would keep (the same argument as i8_filter_tile's), so it costs
// a max and a ballot; the others go through small_tile with the exact dot
// products, after which lo follows the list's (possibly lowered) bound.
template <int METRIC>
__device__ __forceinline__ void small_tile_i8(const KnnArgs& a, const intx16& acc, const float* tn, const int32_t* tr,
                                              const int32_t* th, int tbase, int h, bool qvalid, float qn,
                                              const QueryState& st, SmallList& L, int32_t& lo)
{
    int32_t vmax = INT_MIN;
#pragma unroll
    for (int r = 0; r < 16; r += 2) vmax = max(vmax, max(acc[r], acc[r + 1]));
    if (!__ballot(qvalid && vmax >= lo)) return;
    intx16 dot;
#pragma unroll
    for (int g = 0; g < 4; ++g) {
        const int4 hv = *reinterpret_cast<const int4*>(th + 8 * g + 4 * h);
        const int32_t h4[4] = {hv.x, hv.y, hv.z, hv.w};
#pragma unroll
        for (int e = 0; e < 4; ++e) dot[4 * g + e] = acc[4 * g + e] - h4[e];
    }
    small_tile<METRIC>(a, dot, tn, tr, tbase, h, qvalid, qn, st, L);
    lo = i8_pass_floor<METRIC>(L.kth, qn);
}

// Three waves per SIMD for the list launches (at most 168 VGPRs), two for
// the register short lists.
template <int DP, int METRIC, bool SMALL>
__global__ void __attribute__((amdgpu_flat_work_group_size(256, 256), amdgpu_waves_per_eu(SMALL ? 2 : 3)))
knn_i8_kernel(KnnArgs a)
{
    constexpr int KS = DP / 32;                      // MFMA steps per tile
    constexpr int SUB = I8Stage<DP, SMALL>::SUB;     // tiles per stage
    constexpr int ST = I8Stage<DP, SMALL>::ROWS;     // pool rows per stage
    constexpr int U4_ROW = DP / 16;                  // 16-byte pieces per row
    constexpr int U4_TILE = ST * U4_ROW;
    constexpr int U4_THREAD = (U4_TILE + 255) / 256;
    static_assert(ST <= 256, "one row id per thread");
    static_assert(DP % 32 == 0, "row stride must be a multiple of 32 bytes");
    __shared__ KnnSmemI8<DP, !SMALL> sm;

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

    QueryState st;
    st.seed = FLT_MAX;
    // the seed is read from the output row (the query row unless the item has an out_base)
    const int64_t orow_seed = it.out_base >= 0 ? it.out_base + qlocal : static_cast<int64_t>(qrow);
    if (qvalid && a.seed_d) st.seed = fminf(a.seed_d[orow_seed * a.seed_ld + a.seed_ld - 1], FLT_MAX);
    st.thr = qvalid ? st.seed : -INFINITY;
    st.cnt = 0;
    st.nL = 0;
    st.self = a.exclude_self ? qrow : -2;
    st.orow = it.out_base >= 0 ? it.out_base + qlocal : static_cast<int64_t>(qrow);
    SmallList SL;
    if constexpr (SMALL) {
#pragma unroll
        for (int i = 0; i < kSmallM; ++i) SL.k[i] = kNoKey;
        SL.kth = st.thr;
    } else {
        for (int e = lane; e < kQueriesPerWave * kCB; e += 64) sm.L.buf[w * kQueriesPerWave + e / kCB][e % kCB] = kNoKey;
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

    const int pcount = it.p_count;
    const int ntiles = (pcount + ST - 1) / ST;   // stages
    auto pool_row = [&](int p) -> int32_t {
        if (p >= pcount) return -1;
        p += it.p_rot;
        if (p >= pcount) p -= pcount;
        const int64_t pl = it.p_begin + p;
        return a.p_rows ? a.p_rows[pl] : static_cast<int32_t>(pl);
    };
    auto row_norm = [&](int32_t row) -> float {
        if (row < 0) return INFINITY;
        return METRIC == 0 ? a.np[row] : 0.f;
    };

    // a stage's pool ids: one per row by the threads < ST (two stages
    // ahead), handed to every thread's row requests through LDS
    uint4 pre[U4_THREAD];
    int32_t rid_next = -1;
    auto load_rows = [&](const int32_t* ids) {
#pragma unroll
        for (int u = 0; u < U4_THREAD; ++u) {
            const int e = tid + 256 * u;
            const int32_t id = e < U4_TILE ? ids[e / U4_ROW] : -1;
            const uint4 v = *reinterpret_cast<const uint4*>(a.Xp8 + static_cast<int64_t>(id >= 0 ? id : 0) * DP +
                                                            16 * (e % U4_ROW));
            pre[u] = id >= 0 ? v : make_uint4(0u, 0u, 0u, 0u);
        }
    };
    auto store_rows = [&](int buf) {
#pragma unroll
        for (int u = 0; u < U4_THREAD; ++u) {
            const int e = tid + 256 * u;
            if (e < U4_TILE) *reinterpret_cast<uint4*>(&sm.tile[buf][e / U4_ROW][16 * (e % U4_ROW)]) = pre[u];
        }
    };

    auto row_half = [&](int32_t row, float rn) -> int32_t {
        return row < 0 ? kHalfPast : -(static_cast<int32_t>(rn) >> 1);
    };
    int32_t rid_cur = -1;
    float rn_cur = 0.f;
    if (tid < ST) {
        sm.tnorm[2][tid] = INFINITY; sm.trow[2][tid] = -1; sm.thalf[2][tid] = kHalfPast;
        rid_cur = pool_row(tid);
        sm.sid[0][tid] = rid_cur;
        rn_cur = row_norm(rid_cur);
        rid_next = pool_row(ST + tid);
    }
    __syncthreads();
    load_rows(sm.sid[0]);
    store_rows(0);
    if (tid < ST) {
        sm.trow[0][tid] = rid_cur; sm.tnorm[0][tid] = rn_cur; sm.thalf[0][tid] = row_half(rid_cur, rn_cur);
        sm.sid[1][tid] = rid_next;
    }
    __syncthreads();

    intx16 acc_prev;
#pragma unroll
    for (int r = 0; r < 16; ++r) acc_prev[r] = 0;
    int32_t lo = i8_pass_floor<METRIC>(st.thr, qn);

    // tile (t, u) is filtered while tile (t, u + 1)'s MFMAs run; the last
    // tile of a stage during the first of the next
    auto filter_tile = [&](int slot3, int u, int tbase) {
        const float* tn = &sm.tnorm[slot3][kPoolTile * u];
        const int32_t* tr = &sm.trow[slot3][kPoolTile * u];
        if constexpr (SMALL) {
            small_tile<METRIC>(a, acc_prev, tn, tr, tbase, h, qvalid, qn, st, SL);
        } else {
            i8_filter_tile<METRIC>(sm.L, a, acc_prev, tn, tr, &sm.thalf[slot3][kPoolTile * u], tbase, w, lane, h,
                                   qlocal, qvalid, qn, st, lo);
        }
    };
    for (int t = 0; t < ntiles; ++t) {
        const int buf = t & 1;
        wait_vmem();
        load_rows(sm.sid[(t + 1) & 1]);
        if (tid < ST) {
            rid_cur = rid_next;
            rn_cur = row_norm(rid_cur);
            rid_next = pool_row((t + 2) * ST + tid);
        }

#pragma unroll
        for (int u = 0; u < SUB; ++u) {
            intx16 acc;
            if constexpr (SMALL) {
#pragma unroll
                for (int r = 0; r < 16; ++r) acc[r] = 0;
            } else {
                const int32_t* th = &sm.thalf[t % 3][kPoolTile * u];
#pragma unroll
                for (int g = 0; g < 4; ++g) {
                    const int4 hv = *reinterpret_cast<const int4*>(th + 8 * g + 4 * h);
                    acc[4 * g] = hv.x; acc[4 * g + 1] = hv.y; acc[4 * g + 2] = hv.z; acc[4 * g + 3] = hv.w;
                }
            }
            const int8_t* arow = &sm.tile[buf][kPoolTile * u + j][16 * h];
#pragma unroll
            for (int s = 0; s < KS; ++s) {
                const intx4 av = *reinterpret_cast<const intx4*>(arow + 32 * s);
                acc = __builtin_amdgcn_mfma_i32_32x32x32_i8(av, qf[s], acc, 0, 0, 0);
            }
            // the previous tile: (t, u - 1), or (t - 1, SUB - 1)
            if (u > 0) filter_tile(t % 3, u - 1, t * ST + kPoolTile * (u - 1));
            else if (t > 0) filter_tile((t + 2) % 3, SUB - 1, (t - 1) * ST + kPoolTile * (SUB - 1));
            acc_prev = acc;
        }

        store_rows(buf ^ 1);
        if (tid < ST) {
            sm.trow[(t + 1) % 3][tid] = rid_cur;
            sm.tnorm[(t + 1) % 3][tid] = rn_cur;
            sm.thalf[(t + 1) % 3][tid] = row_half(rid_cur, rn_cur);
            sm.sid[t & 1][tid] = rid_next;   // stage t + 2's ids
        }
        __syncthreads();
    }
    if (ntiles > 0) {
        wait_vmem();
        filter_tile((ntiles - 1) % 3, SUB - 1, (ntiles - 1) * ST + kPoolTile * (SUB - 1));
    }
    if constexpr (SMALL) {
        small_finish(a, SL, j, h, qvalid, st.orow);
    } else {
        wait_vmem();
        merge_queries<false>(sm.L, a, w, lane, __ballot(qvalid && st.cnt > 0) & 0xffffffffull, st);
        if (qvalid) {
            for (int p = st.nL + h; p < a.M; p += 2) {
                a.out_ids[st.orow * a.M + p] = -1;
                a.out_d[st.orow * a.M + p] = INFINITY;
            }
        }
    }
}

// ------------------------------------------------------------ resident pools
//
// Short lists (M <= kSmallM) of every row of a flat query set against a pool
// small enough to sit in LDS: centroid sets of up to resident_rows(Dp) rows
// (C2's top-2 assignment, Lloyd steps and probe table).  Each block loads the
// pool once and then walks query tiles blockIdx.x, + gridDim.x, ...: no stage
// barrier and no row loads inside the scan, the next tile's query bytes in
// flight during the current one.  Tiles go through small_tile_i8 as in
// knn_i8_kernel's short lists (same keys, same order), so the lists are bit
// for bit that kernel's.  (Larger pools split into parts would each warm up
// a list of their own and merge them: measured slower than the staged kernel
// at 2,048 centroids, so they stay there.)
constexpr int kResidentLds = 78 * 1024;   // two blocks per CU

static int resident_rows(int dp) { return kResidentLds / (dp + 28) / kPoolTile * kPoolTile; }

template <int DP, int METRIC>
__global__ void __attribute__((amdgpu_flat_work_group_size(256, 256), amdgpu_waves_per_eu(2)))
knn_i8_resident_kernel(KnnArgs a, int64_t nq, int64_t npool, int pc)   // npool <= pc
{
    constexpr int KS = DP / 32;
    constexpr int RS = DP + 16;          // LDS row stride: rows land on distinct bank groups
    constexpr int U4_ROW = DP / 16;
    extern __shared__ __align__(16) unsigned char res_lds[];
    int8_t* tile = reinterpret_cast<int8_t*>(res_lds);
    float* tn = reinterpret_cast<float*>(res_lds + static_cast<size_t>(pc) * RS);   // |p|^2 (L2), 0 (IP), +inf past the pool
    int32_t* tr = reinterpret_cast<int32_t*>(tn + pc);                            // pool positions, -1 past the pool
    int32_t* th = tr + pc;   // accumulator starts: -floor(|p|^2 / 2) (L2), 0 (IP), kHalfPast past the pool
    const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63, j = lane & 31, h = lane >> 5;
    constexpr int64_t p0 = 0;
    const int pcnt = static_cast<int>(npool);
    for (int e = tid; e < pc * U4_ROW; e += 256) {
        const int r = e / U4_ROW, c = e % U4_ROW;
        uint4 v = make_uint4(0u, 0u, 0u, 0u);
        if (r < pcnt) v = *reinterpret_cast<const uint4*>(a.Xp8 + (p0 + r) * DP + 16 * c);
        *reinterpret_cast<uint4*>(tile + r * RS + 16 * c) = v;
    }
    for (int r = tid; r < pc; r += 256) {
        const float n = r < pcnt ? (METRIC == 0 ? a.np[p0 + r] : 0.f) : INFINITY;
        tn[r] = n;
        tr[r] = r < pcnt ? static_cast<int32_t>(p0 + r) : -1;
        th[r] = r < pcnt ? -(static_cast<int32_t>(n) >> 1) : kHalfPast;
    }
    __syncthreads();
    const int ntiles = (pcnt + kPoolTile - 1) / kPoolTile;
    const int64_t nqt = (nq + kQueriesPerBlock - 1) / kQueriesPerBlock;
    // lane (j, h) holds bytes [32s + 16h, 32s + 16h + 16) of its query for every step s
    auto load_q = [&](int64_t qt, intx4 (&qf)[KS]) {
        const int64_t q = qt * kQueriesPerBlock + w * kQueriesPerWave + j;
        const int8_t* src = a.Xq8 + (q < nq ? q : 0) * DP + 16 * h;
#pragma unroll
        for (int s = 0; s < KS; ++s) {
            const intx4 v = *reinterpret_cast<const intx4*>(src + 32 * s);
#pragma unroll
            for (int e = 0; e < 4; ++e) qf[s][e] = q < nq ? v[e] : 0;
        }
    };
    intx4 qnext[KS];
    int64_t qt = blockIdx.x;
    if (qt < nqt) load_q(qt, qnext);
    for (; qt < nqt; qt += gridDim.x) {
        intx4 qf[KS];
#pragma unroll
        for (int s = 0; s < KS; ++s) qf[s] = qnext[s];
        if (qt + gridDim.x < nqt) load_q(qt + gridDim.x, qnext);
        const int64_t q = qt * kQueriesPerBlock + w * kQueriesPerWave + j;
        const bool qvalid = q < nq;
        const float qn = (qvalid && METRIC == 0) ? a.nq[q] : 0.f;
        QueryState st;
        st.seed = FLT_MAX;
        st.thr = qvalid ? st.seed : -INFINITY;
        st.cnt = 0;
        st.nL = 0;
        st.self = a.exclude_self ? static_cast<int32_t>(q) : -2;
        st.orow = q;
        SmallList SL;
#pragma unroll
        for (int i = 0; i < kSmallM; ++i) SL.k[i] = kNoKey;
        SL.kth = st.thr;
        int32_t lo = i8_pass_floor<METRIC>(st.thr, qn);
        // tile t - 1 is filtered while tile t's MFMAs run
        intx16 acc_prev;
        for (int t = 0; t < ntiles; ++t) {
            intx16 acc;
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                const int4 hv = *reinterpret_cast<const int4*>(th + t * kPoolTile + 8 * g + 4 * h);
                acc[4 * g] = hv.x; acc[4 * g + 1] = hv.y; acc[4 * g + 2] = hv.z; acc[4 * g + 3] = hv.w;
            }
            const int8_t* arow = tile + (t * kPoolTile + j) * RS + 16 * h;
#pragma unroll
            for (int s = 0; s < KS; ++s) {
                const intx4 av = *reinterpret_cast<const intx4*>(arow + 32 * s);
                acc = __builtin_amdgcn_mfma_i32_32x32x32_i8(av, qf[s], acc, 0, 0, 0);
            }
            if (t > 0) {
                const int b = (t - 1) * kPoolTile;
                small_tile_i8<METRIC>(a, acc_prev, tn + b, tr + b, th + b, static_cast<int>(p0) + b, h, qvalid, qn, st,
                                      SL, lo);
            }
            acc_prev = acc;
        }
        if (ntiles > 0) {
            const int b = (ntiles - 1) * kPoolTile;
            small_tile_i8<METRIC>(a, acc_prev, tn + b, tr + b, th + b, static_cast<int>(p0) + b, h, qvalid, qn, st, SL,
                                  lo);
        }
        small_finish(a, SL, j, h, qvalid, st.orow);
    }
}

// ------------------------------------------------------------ wide rows
//
// Rows longer than 256 floats do not fit a wave's registers as a query
// fragment.  The wide kernel accumulates a 32-query x 128-pool-row block per
// wave over chunks of 32 dimensions instead: the pool chunk (128 rows x 32
// dims) is staged through LDS and shared by the block's 4 waves, each wave
// reads its 32 queries' chunk into registers, and the block's four 32x32
// accumulator tiles are filtered once the last chunk is in.  Query rows are
// re-read once per 128 pool rows (from L2 / Infinity Cache).
constexpr int kWideRows = 128;   // pool rows per super-tile
constexpr int kWideChunk = 32;   // dimensions per chunk

struct KnnWideSmem {
    float tile[2][kWideRows][kWideChunk + 4];
    float tnorm[2][kWideRows];
    int32_t trow[2][kWideRows];
    KnnLists L;
};

template <int METRIC>
__global__ void __launch_bounds__(256, 2) knn_wide_kernel(KnnArgs a)
{
    __shared__ KnnWideSmem sm;
    const int per = a.n_items / 8;
    const int item_idx = static_cast<int>(blockIdx.x % 8) * per + static_cast<int>(blockIdx.x / 8);
    if (item_idx >= a.n_items) return;
    const WorkItem it = a.items[item_idx];
    if (it.q_count <= 0) return;

    const int Dp = a.Dp;
    const int nch = Dp / kWideChunk;
    const int tid = threadIdx.x;
    const int w = tid >> 6, lane = tid & 63, j = lane & 31, h = lane >> 5;
    const int qlocal = w * kQueriesPerWave + j;
    const bool qvalid = qlocal < it.q_count;
    const int64_t qi = it.q_begin + qlocal;
    const int32_t qrow = qvalid ? (a.q_rows ? a.q_rows[qi] : static_cast<int32_t>(qi)) : 0;
    const float qn = (qvalid && METRIC == 0) ? a.nq[qrow] : 0.f;

    QueryState st;
    st.seed = FLT_MAX;
    // the seed is read from the output row (the query row unless the item has an out_base)
    const int64_t orow_seed = it.out_base >= 0 ? it.out_base + qlocal : static_cast<int64_t>(qrow);
    if (qvalid && a.seed_d) st.seed = fminf(a.seed_d[orow_seed * a.seed_ld + a.seed_ld - 1], FLT_MAX);
    st.thr = qvalid ? st.seed : -INFINITY;
    st.cnt = 0;
    st.nL = 0;
    st.self = a.exclude_self ? qrow : -2;
    st.orow = it.out_base >= 0 ? it.out_base + qlocal : static_cast<int64_t>(qrow);
    // this wave's 32 buffer rows start empty: every slot holds kNoKey
    for (int e = lane; e < kQueriesPerWave * kCB; e += 64) sm.L.buf[w * kQueriesPerWave + e / kCB][e % kCB] = kNoKey;

    const int pcount = it.p_count;
    const int nst = (pcount + kWideRows - 1) / kWideRows;
    auto pool_row = [&](int p) -> int32_t {
        if (p >= pcount) return -1;
        p += it.p_rot;
        if (p >= pcount) p -= pcount;
        const int64_t pl = it.p_begin + p;
        return a.p_rows ? a.p_rows[pl] : static_cast<int32_t>(pl);
    };
    auto row_norm = [&](int32_t row) -> float {
        if (row < 0) return INFINITY;
        return METRIC == 0 ? a.np[row] : 0.f;
    };

    // thread tid stages float4 (tid & 7) of super-tile rows (tid >> 3) + 32u
    const int c4 = tid & 7, r0 = tid >> 3;
    int32_t rid[4], rid_n[4];
    float4 pre[4];
    auto set_ids = [&](int stile, int32_t (&ids)[4]) {
#pragma unroll
        for (int u = 0; u < 4; ++u) ids[u] = stile < nst ? pool_row(stile * kWideRows + r0 + 32 * u) : -1;
    };
    // chunk c of the current super-tile's rows, or of the next one's
    auto load_pool = [&](bool next, int c) {
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            // rows past the slice stage row 0's values: their norm is +inf and
            // their id -1, so no key of theirs reaches a list (each accumulator
            // element is one pair's own dot product).  Not zeroing them leaves
            // the loads' results untouched until the LDS store at the chunk's
            // end, and the MFMAs run while they are in flight.
            const int32_t id = next ? rid_n[u] : rid[u];
            const float4 v = *reinterpret_cast<const float4*>(a.Xp + static_cast<int64_t>(id >= 0 ? id : 0) * Dp +
                                                              c * kWideChunk + 4 * c4);
            pre[u] = make_float4(v.x, v.y, v.z, v.w);   // a value, not a copy through private memory
        }
    };
    auto store_pool = [&](int buf) {
#pragma unroll
        for (int u = 0; u < 4; ++u) *reinterpret_cast<float4*>(&sm.tile[buf][r0 + 32 * u][4 * c4]) = pre[u];
    };
    // query chunk c: dims c*32 + h*16 + [0, 16)
    const float* qsrc = a.Xq + static_cast<int64_t>(qrow) * Dp + h * (kWideChunk / 2);
    float4 qc[4], qx[4];
    auto load_q = [&](int c, float4 (&dst)[4]) {
#pragma unroll
        for (int s = 0; s < 4; ++s) {   // row 0 for an invalid query: its column is never read
            const float4 v = *reinterpret_cast<const float4*>(qsrc + c * kWideChunk + 4 * s);
            dst[s] = make_float4(v.x, v.y, v.z, v.w);
        }
    };

    set_ids(0, rid);
    set_ids(1, rid_n);
    if (tid < kWideRows) {
        const int32_t r = pool_row(tid);
        sm.trow[0][tid] = r;
        sm.tnorm[0][tid] = row_norm(r);
    }
    load_pool(false, 0);
    store_pool(0);
    load_q(0, qc);
    __syncthreads();

    int g = 0;
    for (int stile = 0; stile < nst; ++stile) {
        floatx16 acc[4];
#pragma unroll
        for (int u = 0; u < 4; ++u)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[u][r] = 0.f;
        // ids and norms of the next super-tile's rows (read by its filter)
        int32_t nrow = -1;
        float nnrm = INFINITY;
        if (tid < kWideRows && stile + 1 < nst) {
            nrow = pool_row((stile + 1) * kWideRows + tid);
            nnrm = row_norm(nrow);
        }
        for (int c = 0; c < nch; ++c) {
            const int buf = g & 1;
            const bool last = c + 1 == nch;
            // the item's last chunk stages row 0 (the ids past the last
            // super-tile are -1) into the buffer no wave reads again
            load_pool(last, last ? 0 : c + 1);
            load_q(last ? 0 : c + 1, qx);
            // the next chunk's loads stay ahead of this chunk's MFMAs (left
            // to itself the scheduler sinks them below the MFMAs, and the LDS
            // store then waits out their whole latency every chunk)
            __builtin_amdgcn_sched_barrier(0);
            // A = pool row u*32 + (lane%32), B = query lane%32, k = dims h*16 + s.
            // Each chunk is summed on its own and added to the running dot:
            // the rounding error grows with sqrt(chunks) instead of sqrt(D/2).
            const float* arow = &sm.tile[buf][j][h * (kWideChunk / 2)];
            floatx16 part[4];
#pragma unroll
            for (int u = 0; u < 4; ++u)
#pragma unroll
                for (int r = 0; r < 16; ++r) part[u][r] = 0.f;
#pragma unroll
            for (int s = 0; s < 4; ++s) {
#pragma unroll
                for (int u = 0; u < 4; ++u) {
                    const float4 av = *reinterpret_cast<const float4*>(arow + u * 32 * (kWideChunk + 4) + 4 * s);
                    part[u] = __builtin_amdgcn_mfma_f32_32x32x2f32(av.x, qc[s].x, part[u], 0, 0, 0);
                    part[u] = __builtin_amdgcn_mfma_f32_32x32x2f32(av.y, qc[s].y, part[u], 0, 0, 0);
                    part[u] = __builtin_amdgcn_mfma_f32_32x32x2f32(av.z, qc[s].z, part[u], 0, 0, 0);
                    part[u] = __builtin_amdgcn_mfma_f32_32x32x2f32(av.w, qc[s].w, part[u], 0, 0, 0);
                }
            }
#pragma unroll
            for (int u = 0; u < 4; ++u)
#pragma unroll
                for (int r = 0; r < 16; ++r) acc[u][r] += part[u][r];
            store_pool(buf ^ 1);
            __syncthreads();
#pragma unroll
            for (int s = 0; s < 4; ++s) qc[s] = qx[s];
            ++g;
        }
        if (tid < kWideRows) {
            sm.trow[(stile + 1) & 1][tid] = nrow;
            sm.tnorm[(stile + 1) & 1][tid] = nnrm;
        }
#pragma unroll
        for (int u = 0; u < 4; ++u) rid[u] = rid_n[u];
        set_ids(stile + 2, rid_n);

        const int sb = stile & 1;
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            wait_vmem();   // list rows stored by this wave's previous merges
            float mkey = INFINITY;
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int i = 8 * (r >> 2) + 4 * h + (r & 3);
                const float pn = sm.tnorm[sb][u * 32 + i];
                mkey = fminf(mkey, METRIC == 0 ? fmaf(-2.f, acc[u][r], pn + qn) : fmaf(-1.f, acc[u][r], pn));
            }
            if (__ballot(mkey <= st.thr))
                tile_append<METRIC, true>(sm.L, a, acc[u], &sm.tnorm[sb][u * 32], &sm.trow[sb][u * 32],
                                    stile * kWideRows + u * 32, w, lane, h, qlocal, qvalid, qn, st);
        }
    }

    wait_vmem();
    merge_queries<true>(sm.L, a, w, lane, __ballot(qvalid && st.cnt > 0) & 0xffffffffull, st);
    if (qvalid) {
        for (int p = st.nL + h; p < a.M; p += 2) {
            a.out_ids[st.orow * a.M + p] = -1;
            a.out_d[st.orow * a.M + p] = INFINITY;
        }
    }
}

// Merges `splits` sorted partial lists per query (rows s*nq + q of parts)
// into rows out_base + q.  One wave per query; lists staged in LDS.
constexpr int kMergeMaxEntries = 2048;
__global__ void __launch_bounds__(64) merge_partials_kernel(const int32_t* __restrict__ pids,
                                                            const float* __restrict__ pd, int64_t nq,
                                                            int splits, int M, int32_t* out_ids,
                                                            float* out_d)
{
    __shared__ float sd[kMergeMaxEntries];
    __shared__ int32_t si[kMergeMaxEntries];
    __shared__ int scount[64];
    const int64_t q = blockIdx.x;
    if (q >= nq) return;
    const int lane = threadIdx.x;
    const int total = splits * M;
    for (int e = lane; e < total; e += 64) {
        const int s = e / M, idx = e % M;
        const int32_t id = pids[(static_cast<int64_t>(s) * nq + q) * M + idx];
        sd[e] = id >= 0 ? pd[(static_cast<int64_t>(s) * nq + q) * M + idx] : INFINITY;
        si[e] = id >= 0 ? id : INT_MAX;
    }
    __syncthreads();
    int valid = 0;
    for (int e = lane; e < total; e += 64) valid += si[e] != INT_MAX;
    scount[lane] = valid;
    __syncthreads();
    int nvalid = 0;
    for (int l = 0; l < 64; ++l) nvalid += scount[l];
    for (int e = lane; e < total; e += 64) {
        if (si[e] == INT_MAX) continue;
        const int s = e / M, idx = e % M;
        int rank = idx;
        for (int s2 = 0; s2 < splits; ++s2)
            if (s2 != s) rank += lower_bound_lds(sd + s2 * M, si + s2 * M, M, sd[e], si[e]);
        if (rank < M) {
            out_ids[q * M + rank] = si[e];
            out_d[q * M + rank] = sd[e];
        }
    }
    for (int p = nvalid + lane; p < M; p += 64) {
        out_ids[q * M + p] = -1;
        out_d[q * M + p] = INFINITY;
    }
}

template <int METRIC, bool SMALL>
static void launch_knn_fused_v(const KnnArgs& a, dim3 grid, hipStream_t stream)
{
    switch (a.Dp) {
    case 32:  hipLaunchKernelGGL((knn_fused_kernel<32, METRIC, SMALL>), grid, dim3(256), 0, stream, a); break;
    case 64:  hipLaunchKernelGGL((knn_fused_kernel<64, METRIC, SMALL>), grid, dim3(256), 0, stream, a); break;
    case 96:  hipLaunchKernelGGL((knn_fused_kernel<96, METRIC, SMALL>), grid, dim3(256), 0, stream, a); break;
    case 128: hipLaunchKernelGGL((knn_fused_kernel<128, METRIC, SMALL>), grid, dim3(256), 0, stream, a); break;
    case 160: hipLaunchKernelGGL((knn_fused_kernel<160, METRIC, SMALL>), grid, dim3(256), 0, stream, a); break;
    case 192: hipLaunchKernelGGL((knn_fused_kernel<192, METRIC, SMALL>), grid, dim3(256), 0, stream, a); break;
    case 224:
        if constexpr (!SMALL) hipLaunchKernelGGL((knn_fused_kernel<224, METRIC, false>), grid, dim3(256), 0, stream, a);
        else GT_REQUIRE(false, "short lists in registers: rows up to 192");
        break;
    case 256:
        if constexpr (!SMALL) hipLaunchKernelGGL((knn_fused_kernel<256, METRIC, false>), grid, dim3(256), 0, stream, a);
        else GT_REQUIRE(false, "short lists in registers: rows up to 192");
        break;
    default:
        GT_REQUIRE(a.Dp % kWideChunk == 0 && a.Dp > 256, "padded dimension " + std::to_string(a.Dp) + " not supported");
        hipLaunchKernelGGL((knn_wide_kernel<METRIC>), grid, dim3(256), 0, stream, a);
        break;
    }
}

template <int METRIC>
static void launch_knn_metric(const KnnArgs& a, dim3 grid, hipStream_t stream)
{
    // register lists would spill beside the query fragments of rows longer
    // than 192: those keep the LDS-buffer path (with its short-list merge)
    if (a.M <= kSmallM && a.Dp <= 192) launch_knn_fused_v<METRIC, true>(a, grid, stream);
    else launch_knn_fused_v<METRIC, false>(a, grid, stream);
}

// SMALL: lists of at most kSmallM entries (assignment against centroids);
// the other variant keeps its registers below the three-wave limit.
template <int METRIC, bool SMALL>
static void launch_knn_i8_v(const KnnArgs& a, dim3 grid, hipStream_t stream)
{
    switch (a.Dp) {
    case 32:  hipLaunchKernelGGL((knn_i8_kernel<32, METRIC, SMALL>), grid, dim3(256), 0, stream, a); break;
    case 64:  hipLaunchKernelGGL((knn_i8_kernel<64, METRIC, SMALL>), grid, dim3(256), 0, stream, a); break;
    case 96:  hipLaunchKernelGGL((knn_i8_kernel<96, METRIC, SMALL>), grid, dim3(256), 0, stream, a); break;
    case 128: hipLaunchKernelGGL((knn_i8_kernel<128, METRIC, SMALL>), grid, dim3(256), 0, stream, a); break;
    case 160: hipLaunchKernelGGL((knn_i8_kernel<160, METRIC, SMALL>), grid, dim3(256), 0, stream, a); break;
    case 192: hipLaunchKernelGGL((knn_i8_kernel<192, METRIC, SMALL>), grid, dim3(256), 0, stream, a); break;
    case 224: hipLaunchKernelGGL((knn_i8_kernel<224, METRIC, SMALL>), grid, dim3(256), 0, stream, a); break;
    case 256: hipLaunchKernelGGL((knn_i8_kernel<256, METRIC, SMALL>), grid, dim3(256), 0, stream, a); break;
    default: GT_REQUIRE(false, "int8 kernel: padded dimension " + std::to_string(a.Dp) + " not supported");
    }
}

template <int METRIC>
static void launch_knn_i8(const KnnArgs& a, dim3 grid, hipStream_t stream)
{
    if (a.M <= kSmallM) launch_knn_i8_v<METRIC, true>(a, grid, stream);
    else launch_knn_i8_v<METRIC, false>(a, grid, stream);
}

// Whether knn_i8_resident_kernel takes the flat job a against np pool rows:
// int8 operands, short lists, identity query and pool lists, no seed, and a
// pool that fits the LDS.
bool resident_supported(const KnnArgs& a, int64_t np)
{
    return a.Xq8 && a.Xp8 && a.M >= 1 && a.M <= kSmallM && !a.q_rows && !a.p_rows && !a.seed_d && a.Dp % 32 == 0 &&
           a.Dp >= 32 && a.Dp <= 256 && np >= 1 && np <= resident_rows(a.Dp);
}

void launch_knn_resident(const KnnArgs& a, int64_t nq, int64_t np, hipStream_t stream)
{
    GT_REQUIRE(resident_supported(a, np), "resident short-list kNN: unsupported job");
    if (nq <= 0) return;
    const int pc = static_cast<int>(ceil_div(np, kPoolTile) * kPoolTile);
    const int64_t nqt = ceil_div(nq, kQueriesPerBlock);
    const dim3 grid(static_cast<unsigned>(std::max<int64_t>(1, std::min<int64_t>(nqt, 1024))));
    const size_t lds = static_cast<size_t>(pc) * (a.Dp + 16) + static_cast<size_t>(pc) * 12;
#define GT_RES(DPV, MET)                                                                                  \
    do {                                                                                                  \
        const void* f = reinterpret_cast<const void*>(&knn_i8_resident_kernel<DPV, MET>);                 \
        GT_HIP(hipFuncSetAttribute(f, hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(lds))); \
        hipLaunchKernelGGL((knn_i8_resident_kernel<DPV, MET>), grid, dim3(256), lds, stream, a, nq, np, pc); \
    } while (0)
#define GT_RES_DP(MET)                                                        \
    switch (a.Dp) {                                                           \
    case 32: GT_RES(32, MET); break;                                          \
    case 64: GT_RES(64, MET); break;                                          \
    case 96: GT_RES(96, MET); break;                                          \
    case 128: GT_RES(128, MET); break;                                        \
    case 160: GT_RES(160, MET); break;                                        \
    case 192: GT_RES(192, MET); break;                                        \
    case 224: GT_RES(224, MET); break;                                        \
    default: GT_RES(256, MET); break;                                         \
    }
    if (a.metric == 0) GT_RES_DP(0) else GT_RES_DP(1)
#undef GT_RES_DP
#undef GT_RES
    GT_HIP(hipGetLastError());
}

// n_items must be a multiple of 8 (XCD-major layout, see knn_fused_kernel).
void launch_knn_fused(const KnnArgs& a, hipStream_t stream)
{
    if (a.n_items <= 0) return;
    GT_REQUIRE(a.M >= 1 && a.M <= kMaxM, "list length must be in [1, 128]");
    GT_REQUIRE(a.n_items % 8 == 0, "work list must be padded to a multiple of 8");
    const dim3 grid(static_cast<unsigned>(a.n_items));
    if (a.Xq8 && a.Xp8) {
        if (a.metric == 0) launch_knn_i8<0>(a, grid, stream);
        else launch_knn_i8<1>(a, grid, stream);
    } else if (a.metric == 0) {
        launch_knn_metric<0>(a, grid, stream);
    } else {
        launch_knn_metric<1>(a, grid, stream);
    }
    GT_HIP(hipGetLastError());
}

void launch_merge_partials(const int32_t* pids, const float* pd, int64_t nq, int splits, int M,
                           int32_t* out_ids, float* out_d, hipStream_t stream)
{
    if (nq <= 0) return;
    GT_REQUIRE(static_cast<int64_t>(splits) * M <= kMergeMaxEntries, "too many partial lists");
    hipLaunchKernelGGL(merge_partials_kernel, dim3(static_cast<unsigned>(nq)), dim3(64), 0, stream, pids, pd,
                       nq, splits, M, out_ids, out_d);
    GT_HIP(hipGetLastError());
}

}  // namespace gtann
