// revmerge_kernels.hip -- reverse-edge merge of a forward graph (Method E,
// rank order: src/optimize_chunked.cu:372-407, 1421-1471,
// src/edge_chunk_accumulator.hpp:471-494) in two kernels on gfx950.
//
// For every destination row j the result is
//   S ++ R ++ (O minus the first occurrence of each element of R), cut to K,
// with S = fwd[j][0..P) (P = K/2, protected), O = fwd[j][P..K), and R the
// distinct sources i of edges i -> j that are not in S, at most L = K - P of
// them, by ascending (rank of j in fwd[i], i) -- the fixed point of the
// reference's weakest-first move-to-front insertion.
//
// (1) rv_scatter_kernel: each block owns the edges of a contiguous range of
//     source rows (at most 32,704 edges, 32 per thread, held in registers).
//     LDS atomics count them per destination bin (2^cshift consecutive
//     rows); a scan of the counts gives the runs' offsets, a second round of
//     atomics places every edge, as a 32-bit key
//       (row within bin << (kbits + sbits)) | (rank << sbits) | (source within block),
//     at its run's cursor in an LDS stage, and the stage leaves as one
//     coalesced copy into the block's own region of `part` (runs in bin
//     order).  The runs' 16-bit offsets (plus the block's total) go to one
//     row of `meta_blk` per block, written contiguously; a tiled transpose
//     turns them bin-major (`meta`), so each merge block reads its offsets
//     as two contiguous rows.
// (2) rv_merge_kernel: one block per bin, bins dealt XCD-major so that
//     neighbouring bins -- whose runs and offsets share cache lines -- run on
//     one XCD.  Fast path (a bin whose keys fit the registers and the LDS):
//     every thread loads a strided share of the bin's keys (consecutive lanes
//     read consecutive keys of the concatenated runs), counts them per (row,
//     rank group) with one LDS atomic each (keeping the returned slot; the
//     counters overlay the run tables, which are dead by then), and after a
//     scan writes each key, as (rank << nbits) | source, to its slot: each
//     row's keys in ascending rank groups.  Then lane t merges row t: the
//     keys stream through a sorted register list of the L strongest
//     non-protected keys (a key at or above the list's L-th costs one
//     compare), and the scan stops once the list's L-th is at or below the
//     floor of the next key's group, so a lane reads about L keys whatever
//     the row's in-degree; the output row is written straight to `out`.
//     Bins beyond the fast path's LDS go to rv_big_kernel (larger blocks);
//     larger ones still take passes over row ranges whose keys fit the LDS,
//     re-reading the runs; a single row beyond the capacity, or one with a
//     repeated source, goes to rv_slow_kernel.
// Larger graphs (beyond 2^21 rows) would give a (bin, block) run table with
// about one key per run, so they take two levels: (1) groups by superbin
// (2^sshift rows) instead of bin, (1b) rv_scatter2_kernel regroups each
// superbin's runs of F consecutive blocks by bin into blocks of its own, and
// (2) merges from those, each superbin's run table transposed on its own.
#include "gtann_common.hpp"

#include <algorithm>
#include <map>
#include <mutex>

namespace gtann {

constexpr int kRvScatterThreads = 1024;
constexpr int kRvEdgesPerThread = 32;     // a scatter block's edges stay in registers
constexpr int kRvMaxBlockEdges = 32704;   // its keys plus 8,192 bin counters fill the 160 KB of LDS
constexpr int kRvMaxBins = 8192;          // LDS counters of the scatter
constexpr int kRvMaxBinShift = 11;        // rows per bin <= 2048
// merge fast path: a bin's keys held in registers, per thread of a block of
// rp threads (a bin of rp rows holds K keys per thread on average; the
// 512-thread blocks of the deferred bins hold up to 512 * 36)
__host__ __device__ constexpr int rv_kpt(int kmax, int rp) { return kmax > 32 && rp < 512 ? 60 : 36; }
constexpr int kRvLdsPerBlock = 40960;     // merge LDS for 4 blocks per CU (degree <= 32; twice that above,
                                          // where the registers allow 2 blocks of 256 threads)
constexpr int kRvGroupBits = 2;
constexpr int kRvGroups = 1 << kRvGroupBits;   // rank groups per row in the merge's LDS grouping
constexpr bool kRvDefer = true;           // bins beyond the fast path go to rv_big_kernel
constexpr int kRvBigThreads = 512;        // blocks of the deferred large bins

// Exclusive scan of a[0..n) in LDS by a block of T threads; returns the
// total (every thread).  wsum: T/64 + 1 words of LDS.
template <int T>
__device__ uint32_t block_exclusive_scan(uint32_t* a, int n, uint32_t* wsum)
{
    const int t = threadIdx.x, lane = t & 63, w = t >> 6;
    const int per = (n + T - 1) / T;
    const int s0 = t * per;
    uint32_t loc = 0;
    for (int q = 0; q < per; ++q)
        if (s0 + q < n) loc += a[s0 + q];
    uint32_t inc = loc;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const uint32_t x = __shfl_up(inc, o);
        if (lane >= o) inc += x;
    }
    if (lane == 63) wsum[w] = inc;
    __syncthreads();
    if (t == 0) {
        uint32_t run = 0;
        for (int q = 0; q < T / 64; ++q) {
            const uint32_t v = wsum[q];
            wsum[q] = run;
            run += v;
        }
        wsum[T / 64] = run;
    }
    __syncthreads();
    uint32_t run = wsum[w] + inc - loc;
    for (int q = 0; q < per; ++q)
        if (s0 + q < n) {
            const uint32_t c = a[s0 + q];
            a[s0 + q] = run;
            run += c;
        }
    const uint32_t total = wsum[T / 64];
    __syncthreads();
    return total;
}

// x = q*K + r for x < 2^24 (float reciprocal, one correction step)
__device__ __forceinline__ void divmod_small(uint32_t x, uint32_t K, float rK, uint32_t& q, uint32_t& r)
{
    q = static_cast<uint32_t>(static_cast<float>(x) * rK);
    if (q * K > x) --q;
    else if ((q + 1) * K <= x) ++q;
    r = x - q * K;
}

__global__ void __launch_bounds__(kRvScatterThreads) rv_scatter_kernel(
    const uint32_t* __restrict__ fwd, int64_t N, int K, int64_t spb, int cshift, int nbins, int kbits, int sbits,
    uint32_t* __restrict__ part, uint16_t* __restrict__ meta, int* __restrict__ err, uint32_t* __restrict__ slow_count)
{
    constexpr int T = kRvScatterThreads;
    constexpr int U = kRvEdgesPerThread;
    extern __shared__ uint32_t lds[];
    uint32_t* cnt = lds;             // nbins counters, then the runs' cursors
    uint32_t* stage = lds + nbins;   // the block's keys in bin order
    __shared__ uint32_t wsum[T / 64 + 1];
    const int t = threadIdx.x;
    if (blockIdx.x == 0 && t == 0) *slow_count = 0u;   // read by the merge and slow kernels after this one
    for (int i = t; i < nbins; i += T) cnt[i] = 0u;
    __syncthreads();
    const int64_t i0 = static_cast<int64_t>(blockIdx.x) * spb;
    const int64_t i1 = i0 + spb < N ? i0 + spb : N;
    const uint32_t ne = static_cast<uint32_t>((i1 - i0) * K);   // <= kRvMaxBlockEdges
    const uint32_t* src = fwd + i0 * K;
    const uint32_t uN = static_cast<uint32_t>(N);
    uint32_t v[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
        const uint32_t e = t + u * T;
        v[u] = e < ne ? src[e] : uN;
    }
    bool bad = false;
#pragma unroll
    for (int u = 0; u < U; ++u) {
        if (v[u] < uN) atomicAdd(&cnt[v[u] >> cshift], 1u);
        else bad |= t + u * T < ne;
    }
    if (bad) atomicExch(err, 1);
    __syncthreads();
    const uint32_t total = block_exclusive_scan<T>(cnt, nbins, wsum);
    uint16_t* mrow = meta + static_cast<int64_t>(blockIdx.x) * (nbins + 1);
    for (int i = t; i < nbins; i += T) mrow[i] = static_cast<uint16_t>(cnt[i]);
    if (t == 0) mrow[nbins] = static_cast<uint16_t>(total);
    __syncthreads();   // the offsets are read before the placement advances them
    const uint32_t rmask = (1u << cshift) - 1u;
    const int hs = kbits + sbits;
    const float rK = 1.0f / static_cast<float>(K);
#pragma unroll
    for (int u = 0; u < U; ++u) {
        if (v[u] >= uN) continue;
        uint32_t il, k;
        divmod_small(t + u * T, static_cast<uint32_t>(K), rK, il, k);
        stage[atomicAdd(&cnt[v[u] >> cshift], 1u)] = ((v[u] & rmask) << hs) | (k << sbits) | il;
    }
    __syncthreads();
    uint32_t* dst = part + i0 * K;
    for (uint32_t q = t; q < total; q += T) dst[q] = stage[q];
}

// meta (block-major, nblk rows of nbins + 1 offsets) -> metaT (bin-major,
// nbins + 1 rows of nblk): each merge block then reads two contiguous rows
// instead of one entry from every block's row.  64 x 64 tiles through LDS;
// blockIdx.z walks the superbins of a two-level merge (one table each).
__global__ void __launch_bounds__(256) rv_meta_transpose_kernel(const uint16_t* __restrict__ meta, int nblk, int nbins,
                                                                uint16_t* __restrict__ metaT,
                                                                uint32_t* __restrict__ big_bins)
{
    __shared__ uint16_t tile[64][65];
    if (blockIdx.x == 0 && blockIdx.y == 0 && blockIdx.z == 0 && threadIdx.x == 0)
        *big_bins = 0u;   // the merge's deferred bins
    const int cols = nbins + 1;
    const int64_t zoff = static_cast<int64_t>(blockIdx.z) * nblk * cols;
    meta += zoff;
    metaT += zoff;
    const int c0 = blockIdx.x * 64, q0 = blockIdx.y * 64;
    const int tx = threadIdx.x & 63, ty = threadIdx.x >> 6;
    for (int r = ty; r < 64; r += 4) {
        const int q = q0 + r, c = c0 + tx;
        if (q < nblk && c < cols) tile[r][tx] = meta[static_cast<int64_t>(q) * cols + c];
    }
    __syncthreads();
    for (int r = ty; r < 64; r += 4) {
        const int c = c0 + r, q = q0 + tx;
        if (q < nblk && c < cols) metaT[static_cast<int64_t>(c) * nblk + q] = tile[tx][r];
    }
}

// Level two of the two-level merge, for graphs whose (bin, block) run table
// would outgrow one level: rv_scatter_kernel has grouped every block's edges
// by superbin (2^sshift destination rows, G of them) with the key layout
// above; block (q2, g) here concatenates superbin g's runs of level-one
// blocks [F q2, F q2 + F) -- at most kRvMaxBlockEdges keys, 32 per thread in
// registers -- and groups them by 2^cshift-row bin into its own region of
// part2 (kRvMaxBlockEdges words; 16-bit run offsets, block-major, in meta2),
// the source now counted from the first row of level-one block F q2 (sbits2
// bits).  A block with more keys sets *err to 2 and leaves its runs empty:
// the caller then merges by another path.
__global__ void __launch_bounds__(kRvScatterThreads) rv_scatter2_kernel(
    const uint32_t* __restrict__ part1, const uint16_t* __restrict__ meta1, int nblk1, int G, int64_t spb, int K,
    int F, int sshift, int cshift, int kbits, int sbits1, int sbits2, uint32_t* __restrict__ part2,
    uint16_t* __restrict__ meta2, int nblk2, int* __restrict__ err)
{
    constexpr int T = kRvScatterThreads;
    constexpr int U = kRvEdgesPerThread;
    extern __shared__ uint32_t lds[];
    const int nb = 1 << (sshift - cshift);   // bins per superbin
    uint32_t* cnt = lds;                      // nb counters, then the runs' cursors
    uint32_t* rst = cnt + nb;                 // F + 1: run starts in the concatenation
    uint32_t* rof = rst + F + 1;              // F: run offsets in part1
    uint32_t* stage = rof + F;                // the block's keys in bin order
    __shared__ uint32_t wsum[T / 64 + 1];
    const int t = threadIdx.x;
    const int q2 = blockIdx.x, g = blockIdx.y;
    const int q1a = q2 * F;
    const int nr = min(F, nblk1 - q1a);
    const uint32_t region1 = static_cast<uint32_t>(spb * K);
    for (int i = t; i < nb; i += T) cnt[i] = 0u;
    for (int r = t; r < nr; r += T) {
        const uint16_t* m = meta1 + static_cast<int64_t>(q1a + r) * (G + 1) + g;
        const uint32_t o0 = m[0];
        rst[r] = static_cast<uint32_t>(m[1]) - o0;
        rof[r] = static_cast<uint32_t>(q1a + r) * region1 + o0;
    }
    __syncthreads();
    const uint32_t total = block_exclusive_scan<T>(rst, nr, wsum);
    uint16_t* mrow = meta2 + (static_cast<int64_t>(g) * nblk2 + q2) * (nb + 1);
    if (total > static_cast<uint32_t>(kRvMaxBlockEdges)) {   // uniform: every thread leaves
        for (int i = t; i <= nb; i += T) mrow[i] = 0;
        if (t == 0) atomicMax(err, 2);
        return;
    }
    if (t == 0) rst[nr] = total;
    __syncthreads();
    // thread t's keys t + u T: the run of the first by binary search, then
    // forward (empty runs are stepped over)
    int r = 0;
    {
        int hi = nr;
        while (hi - r > 1) {
            const int mid = (r + hi) >> 1;
            if (rst[mid] <= static_cast<uint32_t>(t)) r = mid;
            else hi = mid;
        }
    }
    const int hs1 = kbits + sbits1, hs2 = kbits + sbits2;
    const uint32_t rmask = (1u << cshift) - 1u, kmask = (1u << kbits) - 1u, smask1 = (1u << sbits1) - 1u;
    const uint32_t spb32 = static_cast<uint32_t>(spb);
    // every load issued before any key is decoded (the walk is control flow;
    // a decode beside each load would wait for it): key = the level-one key,
    // bin = its run, then both decoded in place
    uint32_t key[U], bin[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
        const uint32_t e = t + u * T;
        bin[u] = 0xFFFFFFFFu;
        if (e < total) {
            while (rst[r + 1] <= e) ++r;
            bin[u] = static_cast<uint32_t>(r);
            key[u] = part1[rof[r] + (e - rst[r])];
        }
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
        if (bin[u] == 0xFFFFFFFFu) continue;
        const uint32_t k1 = key[u];
        const uint32_t row = k1 >> hs1;   // row within the superbin
        key[u] = ((row & rmask) << hs2) | (((k1 >> sbits1) & kmask) << sbits2) | (bin[u] * spb32 + (k1 & smask1));
        bin[u] = row >> cshift;
    }
#pragma unroll
    for (int u = 0; u < U; ++u)
        if (bin[u] != 0xFFFFFFFFu) atomicAdd(&cnt[bin[u]], 1u);
    __syncthreads();
    block_exclusive_scan<T>(cnt, nb, wsum);
    for (int i = t; i < nb; i += T) mrow[i] = static_cast<uint16_t>(cnt[i]);
    if (t == 0) mrow[nb] = static_cast<uint16_t>(total);
    __syncthreads();   // the offsets are read before the placement advances them
#pragma unroll
    for (int u = 0; u < U; ++u)
        if (bin[u] != 0xFFFFFFFFu) stage[atomicAdd(&cnt[bin[u]], 1u)] = key[u];
    __syncthreads();
    uint32_t* dst = part2 + (static_cast<int64_t>(g) * nblk2 + q2) * kRvMaxBlockEdges;
    for (uint32_t q = t; q < total; q += T) dst[q] = stage[q];
}

// median of three unsigned words in one instruction
__device__ __forceinline__ uint32_t med3_u32(uint32_t x, uint32_t lo, uint32_t hi)
{
    uint32_t r;
    asm("v_med3_u32 %0, %1, %2, %3" : "=v"(r) : "v"(x), "v"(lo), "v"(hi));
    return r;
}

// Sorted insertion of x into the ascending register list a[0..LM):
// a'[l] = clamp(x, a[l-1], a[l]) = med3(x, a[l-1], a[l]) (a[-1] = 0), one
// instruction per slot.
template <int LM>
__device__ __forceinline__ void list_insert(uint32_t (&a)[LM], uint32_t x)
{
#pragma unroll
    for (int l = LM - 1; l >= 1; --l) a[l] = med3_u32(x, a[l - 1], a[l]);
    a[0] = min(a[0], x);
}

// one of 64 bits per id (a filter ahead of exact compares; no multiply)
__device__ __forceinline__ uint64_t bloom_bit(uint32_t v)
{
    return 1ull << ((v ^ (v >> 6) ^ (v >> 12)) & 63u);
}

// Dedup-aware insertion into the lane's sorted list lst[0..L) (LM slots):
// a key at or above the L-th, or of a protected source, is dropped; a source
// already in the list keeps its stronger key.
template <int KMAX>
__device__ __forceinline__ void rv_offer_dedup(uint32_t (&lst)[(KMAX + 1) / 2], uint32_t& worst, uint32_t x,
                                               const uint32_t (&fw)[KMAX], int P, int L, uint32_t gmask,
                                               uint64_t sbloom)
{
    constexpr int LM = (KMAX + 1) / 2;
    if (x >= worst) return;
    const uint32_t s = x & gmask;
    if (sbloom & bloom_bit(s)) {
        bool prot = false;
#pragma unroll
        for (int p = 0; p < KMAX / 2; ++p) prot |= (p < P) && fw[p] == s;
        if (prot) return;
    }
    int at = -1;
#pragma unroll
    for (int l = 0; l < LM; ++l)
        if (at < 0 && l < L && lst[l] != 0xFFFFFFFFu && (lst[l] & gmask) == s) at = l;
    if (at >= 0) {
        bool weaker = false;   // the listed key is weaker than x
#pragma unroll
        for (int l = 0; l < LM; ++l)
            if (l == at) weaker = lst[l] > x;
        if (!weaker) return;
#pragma unroll
        for (int l = 0; l < LM - 1; ++l)
            if (l >= at) lst[l] = lst[l + 1];
        lst[LM - 1] = 0xFFFFFFFFu;
    }
    list_insert<LM>(lst, x);
#pragma unroll
    for (int l = 0; l < LM; ++l)
        if (l == L - 1) worst = lst[l];
}

// The merge of one row by one lane from its n grouped LDS keys.  fw: the
// forward row (array entries >= K unused); st: the row's LDS stage, which
// receives the output.  The list has LM slots; its first LM - L hold zero
// keys, so that its last slot is always the L-th real key and no runtime
// bound appears in the per-key loop (protected sources are compared against
// a copy of S padded with a value no source takes).
template <int KMAX>
__device__ __forceinline__ bool rv_merge_lane(const uint32_t (&fw)[KMAX], int K, const uint32_t* grouped, uint32_t n,
                                              int nbits, uint32_t* st, uint32_t gfloor = 0u)
{
    constexpr int LM = (KMAX + 1) / 2;
    constexpr int PM = KMAX / 2;
    const int P = K >> 1, L = K - P;
    const uint32_t gmask = (1u << nbits) - 1u;
    static_assert(PM % 2 == 0, "protected slots in pairs");
    uint32_t S[PM];
#pragma unroll
    for (int p = 0; p < PM; ++p) {
        S[p] = p < P ? fw[p] : 0xFFFFFFFFu;
        // an opaque register copy: the per-key compares below then test
        // plain values instead of re-deriving the uniform bound p < P
        asm volatile("" : "+v"(S[p]));
    }
    uint32_t lst[LM];
#pragma unroll
    for (int l = 0; l < LM; ++l) lst[l] = l < LM - L ? 0u : 0xFFFFFFFFu;
    auto offer = [&](uint32_t x) {
        if (x >= lst[LM - 1]) return;
        // protected: min_p (S[p] ^ s) == 0 (the padding never matches a source)
        const uint32_t s = x & gmask;
        uint32_t m = 0xFFFFFFFFu;
#pragma unroll
        for (int p = 0; p < PM; p += 2) m = min(m, min(S[p] ^ s, S[p + 1] ^ s));
        if (m == 0u) return;
        list_insert<LM>(lst, x);
    };
    // four LDS reads in flight per step.  With the keys in ascending rank
    // groups (gfloor != 0 masks a key down to its group's smallest key), the
    // scan ends once the list's last slot is at or below the floor of the
    // next key's group: no later key can enter.
    uint32_t e = 0;
    for (; e + 4 <= n; e += 4) {
        uint32_t x[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) x[u] = grouped[e + u];
        if (gfloor && lst[LM - 1] <= (x[0] & gfloor)) break;
#pragma unroll
        for (int u = 0; u < 4; ++u) offer(x[u]);
    }
    for (; e < n; ++e) {
        const uint32_t x = grouped[e];
        if (gfloor && lst[LM - 1] <= (x & gfloor)) break;
        offer(x);
    }
    // R = the last L slots.  Rv: each slot's source if it is a real entry of
    // R, else a sentinel of its own (>= 2^31, no source takes it).
    uint32_t Rv[LM];
#pragma unroll
    for (int l = 0; l < LM; ++l) {
        Rv[l] = (l >= LM - L && lst[l] != 0xFFFFFFFFu) ? (lst[l] & gmask) : (0x80000000u + l);
        asm volatile("" : "+v"(Rv[l]));
    }
    // a source twice in R (a forward row that repeats an id): the row goes
    // to the slow kernel
    bool dup = false;
#pragma unroll
    for (int l = 1; l < LM; ++l)
#pragma unroll
        for (int m = 0; m < l; ++m) dup |= Rv[l] == Rv[m];
    if (dup) return false;
    int nR = 0;
#pragma unroll
    for (int l = 0; l < LM; ++l) nR += Rv[l] < 0x80000000u ? 1 : 0;
    // output: S, then R, then O minus the first occurrence of each element of R
#pragma unroll
    for (int p = 0; p < PM; ++p)
        if (p < P) st[p] = fw[p];
#pragma unroll
    for (int l = 0; l < LM; ++l)
        if (Rv[l] < 0x80000000u) st[P + l - (LM - L)] = Rv[l];
    if (nR < L) {
        // Ov: O's entries in place, the rest a value no id takes
        uint32_t Ov[KMAX];
#pragma unroll
        for (int k = 0; k < KMAX; ++k) {
            Ov[k] = (k >= P && k < K) ? fw[k] : 0xFFFFFFFEu;
            asm volatile("" : "+v"(Ov[k]));
        }
        uint64_t rbloom = 0;
#pragma unroll
        for (int l = 0; l < LM; ++l) rbloom |= Rv[l] < 0x80000000u ? bloom_bit(Rv[l]) : 0ull;
        int pos = P + nR;
#pragma unroll
        for (int k = 0; k < KMAX; ++k) {
            const uint32_t o = Ov[k];
            if (o == 0xFFFFFFFEu) continue;
            bool consumed = false;
            if (rbloom & bloom_bit(o)) {
                bool inR = false;
#pragma unroll
                for (int l = 0; l < LM; ++l) inR |= Rv[l] == o;
                if (inR) {
                    bool earlier = false;
#pragma unroll
                    for (int q = 0; q < k; ++q) earlier |= Ov[q] == o;
                    consumed = !earlier;
                }
            }
            if (!consumed && pos < K) st[pos++] = o;
        }
    }
    return true;
}

// rv_merge_lane for K == KMAX, writing the output row orow directly: S =
// fw[0..P) and the list's sources as 16-byte stores (a short list leaves
// its tail slots to the next stores), then, when R is short, the entries of
// O = fw[P..K) that are not the first occurrence in O of an element of R as
// single stores at their positions.  Nothing is written when R repeats a
// source (false: the row goes to the slow kernel).
template <int KMAX>
__device__ __forceinline__ bool rv_merge_full(const uint32_t (&fw)[KMAX], const uint32_t* grouped, uint32_t n,
                                              int nbits, uint32_t* __restrict__ orow, uint32_t gfloor)
{
    constexpr int P = KMAX / 2, L = KMAX - P;
    static_assert(P == L && P % 4 == 0, "even output degree, whole 16-byte halves");
    const uint32_t gmask = (1u << nbits) - 1u;
    uint32_t S[P];
#pragma unroll
    for (int p = 0; p < P; ++p) S[p] = fw[p];
    uint32_t lst[L];
#pragma unroll
    for (int l = 0; l < L; ++l) lst[l] = 0xFFFFFFFFu;
    auto offer = [&](uint32_t x) {
        if (x >= lst[L - 1]) return;
        // protected: some S[p] == s, i.e. min_p (S[p] ^ s) == 0 -- vector
        // instructions only (a wave takes the test whenever one lane needs it)
        const uint32_t s = x & gmask;
        uint32_t m = 0xFFFFFFFFu;
#pragma unroll
        for (int p = 0; p < P; p += 2) m = min(m, min(S[p] ^ s, S[p + 1] ^ s));
        if (m == 0u) return;
        list_insert<L>(lst, x);
    };
    // keys in ascending rank groups: stop once the list's last slot is at or
    // below the floor of the next key's group (x & gfloor)
    uint32_t e = 0;
    for (; e + 8 <= n; e += 8) {
        uint32_t x[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) x[u] = grouped[e + u];
        if (lst[L - 1] <= (x[0] & gfloor)) break;
#pragma unroll
        for (int u = 0; u < 8; ++u) offer(x[u]);
    }
    for (; e < n; ++e) {
        const uint32_t x = grouped[e];
        if (lst[L - 1] <= (x & gfloor)) break;
        offer(x);
    }
    uint32_t Rv[L];
    int nR = 0;
#pragma unroll
    for (int l = 0; l < L; ++l) {
        Rv[l] = lst[l] != 0xFFFFFFFFu ? (lst[l] & gmask) : (0x80000000u + l);
        nR += lst[l] != 0xFFFFFFFFu ? 1 : 0;
    }
    bool dup = false;
#pragma unroll
    for (int l = 1; l < L; ++l)
#pragma unroll
        for (int m = 0; m < l; ++m) dup |= Rv[l] == Rv[m];
    if (dup) return false;
    uint4* o4 = reinterpret_cast<uint4*>(orow);
#pragma unroll
    for (int m = 0; m < P / 4; ++m) o4[m] = make_uint4(fw[4 * m], fw[4 * m + 1], fw[4 * m + 2], fw[4 * m + 3]);
#pragma unroll
    for (int m = 0; m < L / 4; ++m) o4[P / 4 + m] = make_uint4(Rv[4 * m], Rv[4 * m + 1], Rv[4 * m + 2], Rv[4 * m + 3]);
    if (nR < L) {
        // O's entries, minus the first occurrence of each element of R, fill
        // positions P + nR .. K - 1
        uint64_t rbloom = 0;
#pragma unroll
        for (int l = 0; l < L; ++l) rbloom |= l < nR ? bloom_bit(Rv[l]) : 0ull;
        int pos = P + nR;
#pragma unroll
        for (int k = P; k < KMAX; ++k) {
            const uint32_t x = fw[k];
            bool consumed = false;
            if (rbloom & bloom_bit(x)) {
                bool inR = false;
#pragma unroll
                for (int l = 0; l < L; ++l) inR |= Rv[l] == x;
                bool earlier = false;
#pragma unroll
                for (int q = P; q < k; ++q) earlier |= fw[q] == x;
                consumed = inR && !earlier;
            }
            if (!consumed && pos < KMAX) orow[pos] = x;
            pos += consumed ? 0 : 1;
        }
    }
    return true;
}

// One forward row (K words) into registers; entries from K on are unused.
template <int KMAX>
__device__ __forceinline__ void rv_load_row(const uint32_t* __restrict__ g, int K, uint32_t (&fw)[KMAX])
{
    if ((K & 3) == 0) {
        const uint4* g4 = reinterpret_cast<const uint4*>(g);
#pragma unroll
        for (int m = 0; m < KMAX / 4; ++m) {
            const uint4 x = 4 * m < K ? g4[m] : make_uint4(~0u, ~0u, ~0u, ~0u);
            fw[4 * m] = x.x;
            fw[4 * m + 1] = x.y;
            fw[4 * m + 2] = x.z;
            fw[4 * m + 3] = x.w;
        }
    } else {
#pragma unroll
        for (int k = 0; k < KMAX; ++k) fw[k] = k < K ? g[k] : ~0u;
    }
}

// Rows the fast path leaves (keys beyond the LDS capacity, or a source
// repeated in R), as (bin << 11 | row within bin), one wave per row: every
// lane keeps the dedup-aware best L of a strided share of the bin's keys of
// the row; the 64 lists (LDS, 64 * L words) then give R: per source its
// strongest listed key, ranked among all such keys.  A fixed grid walks the
// list; every wave ends when the list is done.
template <int KMAX>
__global__ void __launch_bounds__(256) rv_slow_kernel(const uint32_t* __restrict__ fwd, int64_t N, int K, int nblk,
                                                      int64_t spb, int bsh, uint32_t region, int cshift, int nbins,
                                                      int kbits, int sbits,
                                                      int nbits, const uint32_t* __restrict__ part,
                                                      const uint16_t* __restrict__ meta,
                                                      const uint32_t* __restrict__ slow_rows,
                                                      const uint32_t* __restrict__ slow_count, uint32_t* __restrict__ out)
{
    constexpr int LM = (KMAX + 1) / 2;
    extern __shared__ uint32_t lds[];
    const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int P = K >> 1, L = K - P;
    uint32_t* rs = lds + w * (2 * nblk + 1 + 64 * LM + KMAX + 1);   // run starts (nblk + 1)
    uint32_t* rb = rs + nblk + 1;                                    // run bases (nblk)
    uint32_t* U = rb + nblk;                                         // 64 * L listed keys
    uint32_t* st = U + 64 * LM;                                      // the output row
    const uint32_t gmask = (1u << nbits) - 1u;
    const uint32_t smask = (1u << sbits) - 1u, kmask = (1u << kbits) - 1u;
    const int hs = kbits + sbits;
    const uint32_t cnt = *slow_count;
    for (uint32_t i = blockIdx.x * 4 + w; i < cnt; i += gridDim.x * 4) {
        const uint32_t code = slow_rows[i];
        const int64_t b = code >> 11;
        const uint32_t row = code & 2047u;
        const int64_t j = (b << cshift) + row;
        const int64_t mr = b + (b >> bsh);   // the bin's row of meta
        const uint32_t qb = static_cast<uint32_t>(b >> bsh) * static_cast<uint32_t>(nblk);
        // the bin's runs: starts by a wave scan
        uint32_t carry = 0;
        for (int q0 = 0; q0 < nblk; q0 += 64) {
            const int q = q0 + lane;
            const int qc = q < nblk ? q : 0;
            const uint32_t o0 = meta[mr * nblk + qc];
            const uint32_t c = q < nblk ? static_cast<uint32_t>(meta[(mr + 1) * nblk + qc]) - o0 : 0u;
            uint32_t inc = c;
#pragma unroll
            for (int o = 1; o < 64; o <<= 1) {
                const uint32_t x = __shfl_up(inc, o);
                if (lane >= o) inc += x;
            }
            if (q < nblk) {
                rs[q] = carry + inc - c;
                rb[q] = (qb + static_cast<uint32_t>(q)) * region + o0;
            }
            carry += __shfl(inc, 63);
        }
        if (lane == 0) rs[nblk] = carry;
        wave_sync();
        uint32_t fw[KMAX];
#pragma unroll
        for (int k = 0; k < KMAX; ++k) fw[k] = k < K ? fwd[j * K + k] : 0xFFFFFFFFu;
        uint64_t sbloom = 0;
#pragma unroll
        for (int p = 0; p < KMAX / 2; ++p)
            if (p < P) sbloom |= bloom_bit(fw[p]);
        uint32_t lst[LM];
#pragma unroll
        for (int l = 0; l < LM; ++l) lst[l] = 0xFFFFFFFFu;
        uint32_t worst = 0xFFFFFFFFu;
        for (int t = 0; t < nblk; ++t) {
            const uint32_t len = rs[t + 1] - rs[t];
            const uint32_t* run = part + rb[t];
            const uint32_t sb0 = static_cast<uint32_t>(t * spb);
            for (uint32_t q = lane; q < len; q += 64) {
                const uint32_t key = run[q];
                if ((key >> hs) != row) continue;
                rv_offer_dedup<KMAX>(lst, worst, (((key >> sbits) & kmask) << nbits) | (sb0 + (key & smask)), fw, P,
                                     L, gmask, sbloom);
            }
        }
#pragma unroll
        for (int l = 0; l < LM; ++l)
            if (l < L) U[lane * L + l] = lst[l];
        wave_sync();
        // drop every listed key of a source that has a stronger listed key
        const int nu = 64 * L;
        bool weak[LM];
#pragma unroll
        for (int l = 0; l < LM; ++l) {
            weak[l] = false;
            if (l >= L || lst[l] == 0xFFFFFFFFu) continue;
            const uint32_t s = lst[l] & gmask;
            for (int e = 0; e < nu; ++e) {
                const uint32_t y = U[e];
                weak[l] |= y != 0xFFFFFFFFu && (y & gmask) == s && y < lst[l];
            }
        }
        wave_sync();
#pragma unroll
        for (int l = 0; l < LM; ++l)
            if (l < L && weak[l]) U[lane * L + l] = 0xFFFFFFFFu;
        wave_sync();
        // rank the remaining keys (distinct sources): the first L form R
        int have = 0;
#pragma unroll
        for (int l = 0; l < LM; ++l) {
            if (l >= L || lst[l] == 0xFFFFFFFFu || weak[l]) continue;
            ++have;
            int rank = 0;
            for (int e = 0; e < nu; ++e) rank += U[e] < lst[l] ? 1 : 0;
            if (rank < L) st[P + rank] = lst[l] & gmask;
        }
        int total = have;
#pragma unroll
        for (int o = 32; o >= 1; o >>= 1) total += __shfl_xor(total, o);
        const int nR = total < L ? total : L;
        wave_sync();
        if (lane == 0) {
            for (int p = 0; p < P; ++p) st[p] = fw[p];
            int pos = P + nR;
            for (int k = P; k < K; ++k) {
                const uint32_t o = fw[k];
                bool inR = false, earlier = false;
                for (int l = 0; l < nR; ++l) inR |= st[P + l] == o;
                for (int q = P; q < k; ++q) earlier |= fw[q] == o;
                if (!(inR && !earlier) && pos < K) st[pos++] = o;
            }
        }
        wave_sync();
        if (lane < K) out[j * K + lane] = st[lane];
        wave_sync();
    }
}

// LDS words before the row starts: the 16-bit run tables of the key loading
__host__ __device__ inline int rv_head_words(int nblk) { return (2 * nblk + 2) / 2; }

// LDS words before the group buffer: the run tables and the row starts of
// the general path (rows_max + 1), which the fast path's (row, rank group)
// starts (rows_max * kRvGroups + 1, when a bin's rows fit one block of rp
// threads) overlay once the keys are loaded
__host__ __device__ inline int rv_pre_words(int nblk, int cshift, int rp)
{
    const int rows_max = 1 << cshift;
    const int general = rv_head_words(nblk) + rows_max + 1;
    const int fast = rows_max <= rp ? rows_max * kRvGroups + 1 : 0;
    return general > fast ? general : fast;
}

// The merge of bin b by one block of RP threads.  DEFER: a bin that does not
// fit the fast path is appended to big_bins (for rv_big_kernel) instead of
// taking the general path, so that a few long blocks do not trail the launch.
template <int KMAX, int RP, bool DEFER>
__device__ __forceinline__ void rv_merge_bin(int b, const uint32_t* __restrict__ fwd, int64_t N, int K, int nblk,
                                             int64_t spb, int bsh, uint32_t region, int cshift, int nbins, int kbits,
                                             int sbits, int nbits,
                                             const uint32_t* __restrict__ part, const uint16_t* __restrict__ meta,
                                             uint32_t* __restrict__ out, int cap, uint32_t* __restrict__ slow_rows,
                                             uint32_t* __restrict__ slow_count, uint32_t* __restrict__ big_bins,
                                             uint32_t* lds, uint32_t* wsum)
{
    constexpr int KPT = rv_kpt(KMAX, RP);
    constexpr int G = kRvGroups;
    const int t = threadIdx.x;
    const int rows_max = 1 << cshift;
    uint16_t* rs = reinterpret_cast<uint16_t*>(lds);                  // nblk + 1: run starts in the bin's keys
    uint16_t* roff = rs + nblk + 1;                                   // nblk: run offsets in the block regions
    uint32_t* rowst = lds + rv_head_words(nblk);                      // rows_max + 1: row starts (general path)
    uint32_t* cnt = lds;                                              // fast path: (row, group) starts
    uint32_t* grouped = lds + rv_pre_words(nblk, cshift, RP);         // cap: keys grouped by row
    const int64_t j0 = static_cast<int64_t>(b) << cshift;
    const int rows = static_cast<int>(N - j0 < rows_max ? N - j0 : rows_max);
    const int hs = kbits + sbits;
    const uint32_t smask = (1u << sbits) - 1u;
    const uint32_t kmask = (1u << kbits) - 1u;
    // the bin's runs: block regions qb + q of part (qb = 0 with one level)
    const uint32_t qb = static_cast<uint32_t>(b >> bsh) * static_cast<uint32_t>(nblk);
    // ranks per group: 2^gsh (G groups cover every rank below 2^kbits)
    const int gsh = kbits > kRvGroupBits ? kbits - kRvGroupBits : 0;
    // a converted key's group floor: the key with its rank's low gsh bits and its source cleared
    const uint32_t gfloor = ~((1u << (nbits + gsh)) - 1u);

    // run lengths (in the group buffer's space), scanned into starts
    const uint16_t* m0 = meta + static_cast<int64_t>(b + (b >> bsh)) * nblk;   // bin-major: this bin's and the next row
    for (int q = t; q < nblk; q += RP) {
        const uint32_t o0 = m0[q];
        grouped[q] = static_cast<uint32_t>(m0[q + nblk]) - o0;
        roff[q] = static_cast<uint16_t>(o0);
    }
    for (int r = t; r <= rows_max; r += RP) rowst[r] = 0u;
    __syncthreads();
    const uint32_t T = block_exclusive_scan<RP>(grouped, nblk, wsum);
    auto convert = [&](uint32_t key, uint32_t q) {
        return (((key >> sbits) & kmask) << nbits) | (q * static_cast<uint32_t>(spb) + (key & smask));
    };

    if (rows_max <= RP && T <= static_cast<uint32_t>(cap) && T <= static_cast<uint32_t>(RP * KPT)) {
        for (int q = t; q <= nblk; q += RP) rs[q] = static_cast<uint16_t>(q < nblk ? grouped[q] : T);
        __syncthreads();
        // the run of every key (in the group buffer's space)
        for (int q = t; q < nblk; q += RP)
            for (uint32_t e = rs[q]; e < rs[q + 1]; ++e) grouped[e] = static_cast<uint32_t>(q);
        __syncthreads();
        uint32_t qq[KPT], key[KPT];
#pragma unroll
        for (int u = 0; u < KPT; ++u) {
            const uint32_t e = t + u * RP;
            qq[u] = e < T ? grouped[e] : 0u;
        }
#pragma unroll
        for (int u = 0; u < KPT; ++u) {
            const uint32_t e = t + u * RP;
            key[u] = e < T ? part[(qb + qq[u]) * region + roff[qq[u]] + (e - rs[qq[u]])] : 0u;
        }
        // the run tables are dead (every key is loaded): the (row, group)
        // counters go there
        __syncthreads();
        for (int i = t; i <= rows * G; i += RP) cnt[i] = 0u;
        __syncthreads();
        // count per (row, rank group), keeping each key's slot: qq becomes
        // (row * G + group) << 16 | slot, key the converted key
#pragma unroll
        for (int u = 0; u < KPT; ++u) {
            if (t + u * RP < T) {
                const uint32_t rg = (key[u] >> hs) * G + (((key[u] >> sbits) & kmask) >> gsh);
                const uint32_t slot = atomicAdd(&cnt[rg], 1u);
                key[u] = convert(key[u], qq[u]);
                qq[u] = (rg << 16) | slot;
            }
        }
        __syncthreads();
        block_exclusive_scan<RP>(cnt, rows * G, wsum);
#pragma unroll
        for (int u = 0; u < KPT; ++u)
            if (t + u * RP < T) grouped[cnt[qq[u] >> 16] + (qq[u] & 0xFFFFu)] = key[u];
        // the lane's forward row, requested before the barrier
        const int64_t j = j0 + t;
        uint32_t fw[KMAX];
        if (t < rows) rv_load_row<KMAX>(fwd + j * K, K, fw);
        if (t == 0) cnt[rows * G] = T;
        __syncthreads();
        // lane t merges row t: its keys in ascending rank groups, so the
        // scan ends after about L keys whatever the row's in-degree
        if (t < rows) {
            const uint32_t g0 = cnt[t * G];
            const uint32_t* g = grouped + g0;
            const uint32_t n = cnt[(t + 1) * G] - g0;
            bool ok;
            if (K == KMAX) {
                ok = rv_merge_full<KMAX>(fw, g, n, nbits, out + j * K, gfloor);
            } else {
                ok = rv_merge_lane<KMAX>(fw, K, g, n, nbits, out + j * K, gfloor);
            }
            if (!ok) slow_rows[atomicAdd(slow_count, 1u)] = (static_cast<uint32_t>(b) << 11) | static_cast<uint32_t>(t);
        }
        return;
    }
    if (DEFER) {
        if (t == 0) big_bins[1 + atomicAdd(&big_bins[0], 1u)] = static_cast<uint32_t>(b);
        return;
    }

    // larger bins: the run starts stay in the head of the group buffer (32-bit,
    // the bin may hold more than 65,535 keys); every pass loads the bin's keys
    // in the same coalesced order as above (a key's run by binary search) and
    // groups the rows of one range whose keys fit the rest of the buffer
    uint32_t* rs32 = grouped;   // nblk + 1, already the scanned run starts
    if (t == 0) rs32[nblk] = T;
    uint32_t* gbuf = grouped + nblk + 1;
    const int gcap = cap - nblk - 1;
    __syncthreads();
    // the runs of GL keys by GL interleaved binary searches (the last run
    // starting at or before each key), then the GL loads
    constexpr int GL = 8;   // keys loaded together per thread
    int top = 1;
    while (2 * top <= nblk) top *= 2;
    auto load_keys = [&](uint32_t e0, uint32_t (&kk)[GL], uint32_t (&qq)[GL]) {
        int pos[GL];
#pragma unroll
        for (int u = 0; u < GL; ++u) pos[u] = 0;
        for (int w = top; w > 0; w >>= 1) {
#pragma unroll
            for (int u = 0; u < GL; ++u) {
                const int c = pos[u] + w;
                if (c < nblk && rs32[c] <= e0 + u * RP) pos[u] = c;
            }
        }
#pragma unroll
        for (int u = 0; u < GL; ++u) {
            const uint32_t e = e0 + u * RP;
            qq[u] = static_cast<uint32_t>(pos[u]);
            kk[u] = e < T ? part[(qb + qq[u]) * region + roff[pos[u]] + (e - rs32[pos[u]])] : 0u;
        }
    };
    for (uint32_t e0 = t; e0 < T; e0 += GL * RP) {
        uint32_t kk[GL], qq[GL];
        load_keys(e0, kk, qq);
#pragma unroll
        for (int u = 0; u < GL; ++u)
            if (e0 + u * RP < T) atomicAdd(&rowst[kk[u] >> hs], 1u);
    }
    __syncthreads();
    block_exclusive_scan<RP>(rowst, rows, wsum);
    if (t == 0) rowst[rows] = T;
    __syncthreads();
    for (int r0 = 0; r0 < rows;) {
        // the longest row range from r0 whose keys fit (rows >= r0 still hold their starts)
        int lo = r0 + 1, hi = r0 + RP < rows ? r0 + RP : rows;
        while (lo < hi) {
            const int mid = (lo + hi + 1) >> 1;
            if (rowst[mid] - rowst[r0] <= static_cast<uint32_t>(gcap)) lo = mid;
            else hi = mid - 1;
        }
        const int r1 = lo;
        const uint32_t base = rowst[r0];
        const bool giant = rowst[r0 + 1] - base > static_cast<uint32_t>(gcap);
        __syncthreads();   // every thread has read the starts before the placement moves them
        if (giant) {
            if (t == 0) slow_rows[atomicAdd(slow_count, 1u)] = (static_cast<uint32_t>(b) << 11) | r0;
            r0 = r1;
            continue;
        }
        // placement: rowst[r] becomes the end of row r (= the old start of row r + 1)
        for (uint32_t e0 = t; e0 < T; e0 += GL * RP) {
            uint32_t kk[GL], qq[GL];
            load_keys(e0, kk, qq);
#pragma unroll
            for (int u = 0; u < GL; ++u) {
                const int row = static_cast<int>(kk[u] >> hs);
                if (e0 + u * RP < T && row >= r0 && row < r1)
                    gbuf[atomicAdd(&rowst[row], 1u) - base] = convert(kk[u], qq[u]);
            }
        }
        __syncthreads();
        const int r = r0 + t;
        if (r < r1) {
            const uint32_t s0 = r == r0 ? base : rowst[r - 1];
            const int64_t j = j0 + r;
            uint32_t fw[KMAX];
            rv_load_row<KMAX>(fwd + j * K, K, fw);
            if (!rv_merge_lane<KMAX>(fw, K, gbuf + (s0 - base), rowst[r] - s0, nbits, out + j * K))
                slow_rows[atomicAdd(slow_count, 1u)] = (static_cast<uint32_t>(b) << 11) | static_cast<uint32_t>(r);
        }
        __syncthreads();   // the next pass overwrites the groups
        r0 = r1;
    }
}

// One block per bin, bins dealt XCD-major (workgroup ids go to the 8 XCDs
// round robin, so each XCD takes a contiguous range of bins).  Registers
// for 4 waves per SIMD up to degree 32 (the LDS holds 4 blocks per CU).
template <int KMAX, int RP>
__global__ void __launch_bounds__(RP) __attribute__((amdgpu_waves_per_eu(KMAX > 32 ? 2 : 4))) rv_merge_kernel(const uint32_t* __restrict__ fwd, int64_t N, int K, int nblk,
                                                      int64_t spb, int bsh, uint32_t region, int cshift, int nbins,
                                                      int kbits, int sbits,
                                                      int nbits, const uint32_t* __restrict__ part,
                                                      const uint16_t* __restrict__ meta, uint32_t* __restrict__ out,
                                                      int cap, uint32_t* __restrict__ slow_rows,
                                                      uint32_t* __restrict__ slow_count, uint32_t* __restrict__ big_bins)
{
    extern __shared__ uint32_t lds[];
    __shared__ uint32_t wsum[RP / 64 + 1];
    const int per_xcd = (nbins + 7) / 8;
    const int b = (blockIdx.x & 7) * per_xcd + (blockIdx.x >> 3);
    if (b >= nbins) return;
    rv_merge_bin<KMAX, RP, kRvDefer>(b, fwd, N, K, nblk, spb, bsh, region, cshift, nbins, kbits, sbits, nbits, part,
                                     meta, out, cap,
                                 slow_rows, slow_count, big_bins, lds, wsum);
}

// The bins rv_merge_kernel deferred, by blocks of kRvBigThreads threads with
// a larger group buffer (fast path up to 512 * rv_kpt keys as the LDS allows,
// else the general path);
// a fixed grid walks the list, every block ends when it is done.
template <int KMAX>
__global__ void __launch_bounds__(kRvBigThreads) rv_big_kernel(const uint32_t* __restrict__ fwd, int64_t N, int K, int nblk,
                                                      int64_t spb, int bsh, uint32_t region, int cshift, int nbins,
                                                      int kbits, int sbits,
                                                      int nbits, const uint32_t* __restrict__ part,
                                                      const uint16_t* __restrict__ meta, uint32_t* __restrict__ out,
                                                      int cap, uint32_t* __restrict__ slow_rows,
                                                      uint32_t* __restrict__ slow_count,
                                                      const uint32_t* __restrict__ big_bins)
{
    extern __shared__ uint32_t lds[];
    __shared__ uint32_t wsum[kRvBigThreads / 64 + 1];
    const uint32_t n = big_bins[0];
    for (uint32_t i = blockIdx.x; i < n; i += gridDim.x) {
        rv_merge_bin<KMAX, kRvBigThreads, false>(static_cast<int>(big_bins[1 + i]), fwd, N, K, nblk, spb, bsh, region,
                                                 cshift, nbins, kbits, sbits, nbits, part, meta, out, cap, slow_rows,
                                                 slow_count, nullptr, lds, wsum);
        __syncthreads();   // the next bin reuses the LDS
    }
}

// Raises a kernel's dynamic-LDS limit once per (device, kernel, size): the
// attribute call then stays off the launch path of later calls.
static void ensure_lds(const void* kernel, size_t bytes)
{
    static std::mutex mu;
    static std::map<std::pair<int, const void*>, size_t> done;
    int dev = 0;
    GT_HIP(hipGetDevice(&dev));
    std::lock_guard<std::mutex> lk(mu);
    size_t& have = done[{dev, kernel}];
    if (bytes <= have) return;
    GT_HIP(hipFuncSetAttribute(kernel, hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(bytes)));
    have = bytes;
}

static int bits_for(int64_t n)   // bits of the values 0 .. n-1
{
    int b = 0;
    while ((int64_t(1) << b) < n) ++b;
    return b;
}

// LDS of a merge block of rp threads with the plan's group buffer
size_t rv_merge_lds(const RvPlan& p, int rp)
{
    const size_t words = static_cast<size_t>(rv_pre_words(p.nblk, p.cshift, rp)) + p.cap;
    return words * sizeof(uint32_t);
}

// the merge instantiation (KMAX) of output degree K
static int rv_kmax(int K) { return K <= 16 ? 16 : K <= 32 ? 32 : K <= 48 ? 48 : 64; }

// The merge side of a plan (p.rp, p.cshift, p.nblk set): group buffers and
// the LDS checks
static bool rv_plan_merge(RvPlan& p, int K)
{
    // group buffer: an average bin + 1/16, more when 4 blocks per CU still fit
    p.cap = p.rp * K * 17 / 16;
    RvPlan q = p;
    q.cap = 0;
    // (less the static scan words and the LDS allocation granule)
    const int64_t budget = K > 32 && p.rp == 256 ? 2 * kRvLdsPerBlock : kRvLdsPerBlock;
    const int64_t room = (budget - 512 - static_cast<int64_t>(rv_merge_lds(q, p.rp))) / 4;
    p.cap = static_cast<int>(std::max<int64_t>(p.cap, std::min<int64_t>(room, int64_t(p.rp) * rv_kpt(rv_kmax(K), p.rp))));
    // the run lengths are scanned in the group buffer, whose head keeps them
    // in the general path: leave room for the longest rows besides
    p.cap = std::max(p.cap, p.nblk + 1 + 4 * p.rp);
    // deferred bins: larger blocks, two per CU
    const int64_t room_big = (80 * 1024 - 1024 - static_cast<int64_t>(rv_merge_lds(q, kRvBigThreads))) / 4;
    p.cap_big = static_cast<int>(std::min<int64_t>(room_big, int64_t(kRvBigThreads) * rv_kpt(rv_kmax(K), kRvBigThreads)));
    if (p.cap_big < p.cap) return false;
    RvPlan b = p;
    b.cap = p.cap_big;
    return rv_merge_lds(p, p.rp) <= 160 * 1024 && rv_merge_lds(b, kRvBigThreads) <= 160 * 1024;
}

bool rv_plan(int64_t N, int K, RvPlan& p)
{
    if (N < 1 || K < 1 || K > 64) return false;
    const int64_t E = N * K;
    if (E >= (int64_t(1) << 32)) return false;
    p = RvPlan{};
    p.rp = K > 48 ? 128 : 256;
    p.cshift = K > 48 ? 7 : 8;
    while (p.cshift < kRvMaxBinShift && ceil_div(N, int64_t(1) << p.cshift) > kRvMaxBins) ++p.cshift;
    p.nbins = static_cast<int>(ceil_div(N, int64_t(1) << p.cshift));
    if (p.nbins > kRvMaxBins) return false;
    p.spb = std::min<int64_t>(kRvMaxBlockEdges / K, N);
    p.nblk = static_cast<int>(ceil_div(N, p.spb));
    p.kbits = bits_for(K);
    p.sbits = bits_for(p.spb);
    p.nbits = bits_for(N);
    p.region = static_cast<uint32_t>(p.spb * K);
    if (p.cshift + p.kbits + p.sbits > 32) return false;
    if (p.kbits + p.nbits > 31) return false;   // 0xFFFFFFFF stays free as the empty marker
    return rv_plan_merge(p, K);
}

// Two levels: superbins as large as the level-one key allows (and small
// enough that a small graph still gets several), then F level-one blocks per
// level-two block, sized so that a superbin's runs of F blocks fill about
// 60 % of a block when destinations spread evenly.
bool rv_plan2(int64_t N, int K, RvPlan& p)
{
    if (N < 1 || K < 1 || K > 64) return false;
    const int64_t E = N * K;
    if (E >= (int64_t(1) << 32)) return false;
    p = RvPlan{};
    p.two = true;
    p.rp = K > 48 ? 128 : 256;
    p.cshift = K > 48 ? 7 : 8;
    p.kbits = bits_for(K);
    p.nbits = bits_for(N);
    if (p.kbits + p.nbits > 31) return false;
    p.spb1 = std::min<int64_t>(kRvMaxBlockEdges / K, N);
    p.nblk1 = static_cast<int>(ceil_div(N, p.spb1));
    p.sbits1 = bits_for(p.spb1);
    p.sshift = std::min(32 - p.kbits - p.sbits1, std::max(p.cshift + 2, p.nbits - 6));
    if (p.sshift - p.cshift < 1 || p.sshift - p.cshift > 12) return false;
    p.G = static_cast<int>(ceil_div(N, int64_t(1) << p.sshift));
    if (p.G >= kRvMaxBins) return false;
    const double per_run = static_cast<double>(p.spb1) * K * static_cast<double>(int64_t(1) << p.sshift) / N;
    p.F = static_cast<int>(std::max(1.0, std::min(512.0, 0.6 * kRvMaxBlockEdges / per_run)));
    while (p.F > 1 && p.cshift + p.kbits + bits_for(p.F * p.spb1) > 32) --p.F;
    p.spb = p.F * p.spb1;
    p.sbits = bits_for(p.spb);
    if (p.cshift + p.kbits + p.sbits > 32) return false;
    p.nblk = static_cast<int>(ceil_div(p.nblk1, p.F));
    p.bsh = p.sshift - p.cshift;
    p.nbins = static_cast<int>(ceil_div(N, int64_t(1) << p.cshift));
    p.region = kRvMaxBlockEdges;
    if (static_cast<int64_t>(p.G) * p.nblk * kRvMaxBlockEdges >= (int64_t(1) << 32)) return false;
    return rv_plan_merge(p, K);
}

RvSizes rv_sizes(int64_t N, int K, const RvPlan& p)
{
    RvSizes z{};
    if (p.two) {
        const int64_t nb = int64_t(1) << p.bsh;
        z.part = static_cast<size_t>(p.G) * p.nblk * kRvMaxBlockEdges;
        z.meta = static_cast<size_t>(p.G) * p.nblk * (nb + 1);
        z.part1 = static_cast<size_t>(N) * K;
        z.meta1 = static_cast<size_t>(p.nblk1) * (p.G + 1);
    } else {
        z.part = static_cast<size_t>(N) * K;
        z.meta = static_cast<size_t>(p.nbins + 1) * p.nblk;
    }
    return z;
}

void launch_rv(const uint32_t* fwd, int64_t N, int K, const RvPlan& p, const RvBufs& bf, uint32_t* out, int* err,
               uint32_t* slow_rows, uint32_t* slow_count, uint32_t* big_bins, hipStream_t s)
{
    uint32_t* part = bf.part;
    const uint16_t* meta = bf.meta;
    if (p.two) {
        const int nb = 1 << p.bsh;
        const size_t lds1 = (static_cast<size_t>(p.G) + kRvMaxBlockEdges) * sizeof(uint32_t);
        ensure_lds(reinterpret_cast<const void*>(&rv_scatter_kernel), lds1);
        hipLaunchKernelGGL(rv_scatter_kernel, dim3(p.nblk1), dim3(kRvScatterThreads), lds1, s, fwd, N, K, p.spb1,
                           p.sshift, p.G, p.kbits, p.sbits1, bf.part1, bf.meta1, err, slow_count);
        const size_t lds2 = (static_cast<size_t>(nb) + 2 * p.F + 1 + kRvMaxBlockEdges) * sizeof(uint32_t);
        ensure_lds(reinterpret_cast<const void*>(&rv_scatter2_kernel), lds2);
        hipLaunchKernelGGL(rv_scatter2_kernel, dim3(p.nblk, p.G), dim3(kRvScatterThreads), lds2, s, bf.part1, bf.meta1,
                           p.nblk1, p.G, p.spb1, K, p.F, p.sshift, p.cshift, p.kbits, p.sbits1, p.sbits, bf.part,
                           bf.meta_blk, p.nblk, err);
        hipLaunchKernelGGL(rv_meta_transpose_kernel, dim3(static_cast<unsigned>(ceil_div(nb + 1, 64)),
                                                          static_cast<unsigned>(ceil_div(p.nblk, 64)), p.G),
                           dim3(256), 0, s, bf.meta_blk, p.nblk, nb, bf.meta, big_bins);
    } else {
        const size_t lds_s = (static_cast<size_t>(p.nbins) + kRvMaxBlockEdges) * sizeof(uint32_t);
        ensure_lds(reinterpret_cast<const void*>(&rv_scatter_kernel), lds_s);
        hipLaunchKernelGGL(rv_scatter_kernel, dim3(p.nblk), dim3(kRvScatterThreads), lds_s, s, fwd, N, K, p.spb,
                           p.cshift, p.nbins, p.kbits, p.sbits, part, bf.meta_blk, err, slow_count);
        hipLaunchKernelGGL(rv_meta_transpose_kernel, dim3(static_cast<unsigned>(ceil_div(p.nbins + 1, 64)),
                                                          static_cast<unsigned>(ceil_div(p.nblk, 64))),
                           dim3(256), 0, s, bf.meta_blk, p.nblk, p.nbins, bf.meta, big_bins);
    }
    const size_t lds = rv_merge_lds(p, p.rp);
    RvPlan pb = p;
    pb.cap = p.cap_big;
    const size_t lds_big = rv_merge_lds(pb, kRvBigThreads);
    const int grid = 8 * ((p.nbins + 7) / 8);
#define GT_RV_MERGE(KM, R)                                                                                       \
    do {                                                                                                         \
        ensure_lds(reinterpret_cast<const void*>(&rv_merge_kernel<KM, R>), lds);                                 \
        hipLaunchKernelGGL((rv_merge_kernel<KM, R>), dim3(grid), dim3(R), lds, s, fwd, N, K, p.nblk, p.spb,      \
                           p.bsh, p.region, p.cshift, p.nbins, p.kbits, p.sbits, p.nbits, part, meta, out, p.cap, \
                           slow_rows, slow_count, big_bins);                                                     \
        ensure_lds(reinterpret_cast<const void*>(&rv_big_kernel<KM>), lds_big);                                  \
        hipLaunchKernelGGL((rv_big_kernel<KM>), dim3(std::min(p.nbins, 512)), dim3(kRvBigThreads), lds_big, s, fwd, \
                           N, K,                                                                                 \
                           p.nblk, p.spb, p.bsh, p.region, p.cshift, p.nbins, p.kbits, p.sbits, p.nbits, part,   \
                           meta, out, p.cap_big, slow_rows, slow_count, big_bins);                               \
        const size_t lds_w = (2 * static_cast<size_t>(p.nblk) + 1 + 64 * ((KM + 1) / 2) + KM + 1) * 4 * 4;     \
        ensure_lds(reinterpret_cast<const void*>(&rv_slow_kernel<KM>), lds_w);                                   \
        hipLaunchKernelGGL((rv_slow_kernel<KM>), dim3(256), dim3(256), lds_w, s, fwd, N, K, p.nblk, p.spb,       \
                           p.bsh, p.region, p.cshift, p.nbins, p.kbits, p.sbits, p.nbits, part, meta, slow_rows, \
                           slow_count, out);                                                                     \
    } while (0)
    if (K <= 16) GT_RV_MERGE(16, 256);
    else if (K <= 32) GT_RV_MERGE(32, 256);
    else if (K <= 48) GT_RV_MERGE(48, 256);
    else GT_RV_MERGE(64, 128);
#undef GT_RV_MERGE
    GT_HIP(hipGetLastError());
}

}  // namespace gtann
