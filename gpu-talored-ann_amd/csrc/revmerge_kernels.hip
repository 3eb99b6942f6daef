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
//     source rows.  It counts them per destination bin (2^cshift consecutive
//     rows) in LDS, scans the counts, and writes its edges, bin by bin, into
//     its own contiguous region of `part` as 32-bit keys
//       (row within bin << (kbits + sbits)) | (rank << sbits) | (source within block).
//     The region belongs to one block, so its cache lines fill in one XCD's
//     L2 before they are written back.  Per (bin, block) it records the run
//     length and offset (meta_cnt / meta_off, bin-major).
// (2) rv_merge_kernel: one block per bin.  It gathers the bin's runs, counts
//     keys per row, groups them by row in LDS (as (rank << nbits) | source),
//     and then merges one row per lane: the row's keys stream through a sorted
//     register list of the L strongest non-protected keys (a key at or above
//     the list's L-th costs one compare), duplicate sources are resolved
//     after the fact, and the row is written through LDS so that both the
//     forward rows and the output rows move as coalesced blocks.  A bin whose
//     keys exceed the LDS capacity is merged in several passes over row
//     ranges; a single row beyond the capacity reads its keys from the runs.
#include "gtann_common.hpp"

#include <algorithm>
#include <map>
#include <mutex>

namespace gtann {

constexpr int kRvScatterThreads = 512;
// edges staged in LDS per scatter step: 16384 when its LDS (6 bytes per edge
// plus two counters per bin) fits, else 8192
constexpr size_t rv_scatter_lds(int nbins, int sc) { return (2 * static_cast<size_t>(nbins) + sc) * 4 + sc * 2; }
constexpr int kRvMaxBins = 8192;       // LDS counters of the scatter
constexpr int kRvMaxBinShift = 11;     // rows per bin <= 2048 (LDS row counters of the merge)
constexpr int kRvGather = 32;          // keys of a run loaded together by the merge

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

template <int kRvSubChunk>
__global__ void __launch_bounds__(kRvScatterThreads) rv_scatter_kernel(
    const uint32_t* __restrict__ fwd, int64_t N, int K, int64_t spb, int cshift, int nbins, int kbits, int sbits,
    uint32_t* __restrict__ part, uint32_t* __restrict__ meta_cnt, uint32_t* __restrict__ meta_off,
    int* __restrict__ err, uint32_t* __restrict__ slow_count)
{
    constexpr int T = kRvScatterThreads;
    constexpr int U = kRvSubChunk / T;   // edges per thread per sub-chunk
    extern __shared__ uint32_t h[];      // cur[nbins], sub[nbins], stage[kRvSubChunk], sbin[kRvSubChunk] (u16)
    uint32_t* cur = h;
    uint32_t* sub = h + nbins;
    uint32_t* stage = sub + nbins;
    uint16_t* sbin = reinterpret_cast<uint16_t*>(stage + kRvSubChunk);
    __shared__ uint32_t wsum[T / 64 + 1];
    const int t = threadIdx.x;
    const int nblk = gridDim.x;
    if (blockIdx.x == 0 && t == 0) *slow_count = 0u;   // read by the merge and slow kernels after this one
    for (int i = t; i < nbins; i += T) cur[i] = 0u;
    __syncthreads();
    const int64_t i0 = static_cast<int64_t>(blockIdx.x) * spb;
    const int64_t i1 = i0 + spb < N ? i0 + spb : N;
    const uint32_t ne = i1 > i0 ? static_cast<uint32_t>((i1 - i0) * K) : 0u;   // < 2^24
    const uint32_t* src = fwd + i0 * K;
    const uint32_t uN = static_cast<uint32_t>(N);
    // (1) the block's counts per bin
    bool bad = false;
    for (uint32_t e = t; e < ne; e += U * T) {
        uint32_t v[U];
#pragma unroll
        for (int u = 0; u < U; ++u) v[u] = e + u * T < ne ? src[e + u * T] : uN;
#pragma unroll
        for (int u = 0; u < U; ++u) {
            if (e + u * T >= ne) continue;
            if (v[u] >= uN) bad = true;
            else atomicAdd(&cur[v[u] >> cshift], 1u);
        }
    }
    if (bad) atomicExch(err, 1);
    __syncthreads();
    for (int i = t; i < nbins; i += T) meta_cnt[static_cast<int64_t>(i) * nblk + blockIdx.x] = cur[i];
    block_exclusive_scan<T>(cur, nbins, wsum);
    for (int i = t; i < nbins; i += T) meta_off[static_cast<int64_t>(i) * nblk + blockIdx.x] = cur[i];
    __syncthreads();
    // (2) sub-chunk by sub-chunk: keys sorted by bin in LDS, then stored in
    // that order, so the lanes of a store instruction write runs of
    // consecutive words
    const uint32_t rmask = (1u << cshift) - 1u;
    const int hs = kbits + sbits;
    const float rK = 1.0f / static_cast<float>(K);
    uint32_t* dst = part + i0 * K;
    for (uint32_t c0 = 0; c0 < ne; c0 += kRvSubChunk) {
        for (int i = t; i < nbins; i += T) sub[i] = 0u;
        __syncthreads();
        uint32_t v[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const uint32_t e = c0 + t + u * T;
            v[u] = e < ne ? src[e] : uN;
        }
        uint32_t rk[U];
#pragma unroll
        for (int u = 0; u < U; ++u)
            rk[u] = v[u] < uN ? atomicAdd(&sub[v[u] >> cshift], 1u) : 0u;
        __syncthreads();
        const uint32_t nsub = block_exclusive_scan<T>(sub, nbins, wsum);   // sub = start of each bin's keys
#pragma unroll
        for (int u = 0; u < U; ++u) {
            if (v[u] >= uN) continue;
            const uint32_t b = v[u] >> cshift;
            uint32_t il, k;
            divmod_small(c0 + t + u * T, static_cast<uint32_t>(K), rK, il, k);
            const uint32_t pos = sub[b] + rk[u];
            stage[pos] = ((v[u] & rmask) << hs) | (k << sbits) | il;
            sbin[pos] = static_cast<uint16_t>(b);
        }
        __syncthreads();
        for (uint32_t q = t; q < nsub; q += T) {
            const uint32_t b = sbin[q];
            dst[cur[b] + (q - sub[b])] = stage[q];
        }
        __syncthreads();
        // advance the cursors by this sub-chunk's counts
        for (uint32_t q = t; q < nsub; q += T) {
            const uint32_t b = sbin[q];
            if (q + 1 == nsub || sbin[q + 1] != b) cur[b] += q + 1 - sub[b];
        }
        __syncthreads();
    }
}

// Sorted insertion of x into the ascending register list a[0..LM):
// a'[l] = clamp(x, a[l-1], a[l]) (a[-1] = 0).
template <int LM>
__device__ __forceinline__ void list_insert(uint32_t (&a)[LM], uint32_t x)
{
#pragma unroll
    for (int l = LM - 1; l >= 1; --l) a[l] = min(a[l], max(a[l - 1], x));
    a[0] = min(a[0], x);
}

__device__ __forceinline__ uint64_t bloom_bit(uint32_t v)
{
    return 1ull << ((v * 0x9E3779B1u) >> 26);
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
                                              int nbits, uint32_t* st)
{
    constexpr int LM = (KMAX + 1) / 2;
    constexpr int PM = KMAX / 2;
    const int P = K >> 1, L = K - P;
    const uint32_t gmask = (1u << nbits) - 1u;
    uint32_t S[PM];
    uint64_t sbloom = 0;
#pragma unroll
    for (int p = 0; p < PM; ++p) {
        S[p] = p < P ? fw[p] : 0xFFFFFFFFu;
        // an opaque register copy: the per-key compares below then test
        // plain values instead of re-deriving the uniform bound p < P
        asm volatile("" : "+v"(S[p]));
        sbloom |= p < P ? bloom_bit(fw[p]) : 0ull;
    }
    uint32_t lst[LM];
#pragma unroll
    for (int l = 0; l < LM; ++l) lst[l] = l < LM - L ? 0u : 0xFFFFFFFFu;
    auto offer = [&](uint32_t x) {
        if (x >= lst[LM - 1]) return;
        const uint32_t s = x & gmask;
        if (sbloom & bloom_bit(s)) {
            bool prot = false;
#pragma unroll
            for (int p = 0; p < PM; ++p) prot |= S[p] == s;
            if (prot) return;
        }
        list_insert<LM>(lst, x);
    };
    // four LDS reads in flight per step
    uint32_t e = 0;
    for (; e + 4 <= n; e += 4) {
        uint32_t x[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) x[u] = grouped[e + u];
#pragma unroll
        for (int u = 0; u < 4; ++u) offer(x[u]);
    }
    for (; e < n; ++e) offer(grouped[e]);
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

// Loads a wave's wrn consecutive rows of src (K words each, one contiguous
// run) into the wave's LDS stage (row stride K + 1), all loads in flight
// before the LDS stores; and the reverse.
template <int KMAX>
__device__ __forceinline__ void rv_stage_in(const uint32_t* __restrict__ g, int wrn, int K, uint32_t* wst, int lane)
{
    const uint32_t nw = static_cast<uint32_t>(wrn * K);
    const float rK = 1.0f / static_cast<float>(K);
    uint32_t vv[KMAX];
#pragma unroll
    for (int m = 0; m < KMAX; ++m) {
        const uint32_t f = lane + 64u * m;
        vv[m] = f < nw ? g[f] : 0u;
    }
#pragma unroll
    for (int m = 0; m < KMAX; ++m) {
        const uint32_t f = lane + 64u * m;
        if (f >= nw) continue;
        uint32_t rr, c;
        divmod_small(f, static_cast<uint32_t>(K), rK, rr, c);
        wst[rr * (K + 1) + c] = vv[m];
    }
}

template <int KMAX>
__device__ __forceinline__ void rv_stage_out(uint32_t* __restrict__ g, int wrn, int K, const uint32_t* wst, int lane)
{
    const uint32_t nw = static_cast<uint32_t>(wrn * K);
    const float rK = 1.0f / static_cast<float>(K);
#pragma unroll
    for (int m = 0; m < KMAX; ++m) {
        const uint32_t f = lane + 64u * m;
        if (f >= nw) continue;
        uint32_t rr, c;
        divmod_small(f, static_cast<uint32_t>(K), rK, rr, c);
        g[f] = wst[rr * (K + 1) + c];
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
                                                      int64_t spb, int cshift, int kbits, int sbits, int nbits,
                                                      const uint32_t* __restrict__ part,
                                                      const uint32_t* __restrict__ meta_cnt,
                                                      const uint32_t* __restrict__ meta_off,
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
        // the bin's runs: starts by a wave scan
        uint32_t carry = 0;
        for (int q0 = 0; q0 < nblk; q0 += 64) {
            const int q = q0 + lane;
            const uint32_t c = q < nblk ? meta_cnt[b * nblk + q] : 0u;
            uint32_t inc = c;
#pragma unroll
            for (int o = 1; o < 64; o <<= 1) {
                const uint32_t x = __shfl_up(inc, o);
                if (lane >= o) inc += x;
            }
            if (q < nblk) {
                rs[q] = carry + inc - c;
                rb[q] = static_cast<uint32_t>(q * spb * K) + meta_off[b * nblk + q];
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

template <int KMAX, int RP>
__global__ void __launch_bounds__(RP) rv_merge_kernel(const uint32_t* __restrict__ fwd, int64_t N, int K, int nblk,
                                                      int64_t spb, int cshift, int kbits, int sbits, int nbits,
                                                      const uint32_t* __restrict__ part,
                                                      const uint32_t* __restrict__ meta_cnt,
                                                      const uint32_t* __restrict__ meta_off, uint32_t* __restrict__ out,
                                                      int cap, int ubuf, uint32_t* __restrict__ slow_rows,
                                                      uint32_t* __restrict__ slow_count)
{
    constexpr int W = RP / 64;
    extern __shared__ uint32_t lds[];
    __shared__ uint32_t wsum[W + 1];
    const int t = threadIdx.x, w = t >> 6, lane = t & 63;
    const int rows_max = 1 << cshift;
    uint32_t* rstart = lds;                      // nblk + 1
    uint32_t* rbase = rstart + nblk + 1;         // nblk
    uint32_t* rowstart = rbase + nblk;           // rows_max + 1
    uint32_t* cursor = rowstart + rows_max + 1;  // rows_max
    uint32_t* grouped = cursor + rows_max;       // cap
    uint32_t* ubase = grouped + cap;             // ubuf: the bin's keys as read (<= cap of them), later the stages
    const int b = blockIdx.x;
    const int64_t j0 = static_cast<int64_t>(b) << cshift;
    const int rows = static_cast<int>(N - j0 < rows_max ? N - j0 : rows_max);
    const int hs = kbits + sbits;
    const uint32_t smask = (1u << sbits) - 1u;
    const uint32_t kmask = (1u << kbits) - 1u;

    for (int q = t; q < nblk; q += RP) {
        rstart[q] = meta_cnt[static_cast<int64_t>(b) * nblk + q];
        rbase[q] = static_cast<uint32_t>(q * spb * K) + meta_off[static_cast<int64_t>(b) * nblk + q];
    }
    for (int r = t; r < rows; r += RP) rowstart[r] = 0u;
    __syncthreads();
    const uint32_t T = block_exclusive_scan<RP>(rstart, nblk, wsum);
    if (t == 0) rstart[nblk] = T;
    __syncthreads();
    // keys per row, one run per thread, a run's keys loaded together; when
    // the bin's keys fit, they are kept in LDS in run order
    // (only when the whole bin is one pass: the copy's space later holds the stages)
    const bool keep = T <= static_cast<uint32_t>(ubuf) && T <= static_cast<uint32_t>(cap) && rows <= RP;
    for (int q = t; q < nblk; q += RP) {
        const uint32_t len = rstart[q + 1] - rstart[q];
        const uint32_t* run = part + rbase[q];
        const uint32_t at = rstart[q];
        for (uint32_t j = 0; j < len; j += kRvGather) {
            uint32_t kk[kRvGather];
#pragma unroll
            for (int u = 0; u < kRvGather; ++u) kk[u] = j + u < len ? run[j + u] : 0u;
#pragma unroll
            for (int u = 0; u < kRvGather; ++u) {
                if (j + u >= len) continue;
                atomicAdd(&rowstart[kk[u] >> hs], 1u);
                if (keep) ubase[at + j + u] = kk[u];
            }
        }
    }
    __syncthreads();
    block_exclusive_scan<RP>(rowstart, rows, wsum);
    if (t == 0) rowstart[rows] = T;
    __syncthreads();

    const int ST = K + 1;
    uint32_t* wst = ubase + w * 64 * ST;
    for (int r0 = 0; r0 < rows;) {
        // the longest row range from r0 whose keys fit in LDS; a row beyond
        // the capacity goes to the slow kernel
        int lo = r0 + 1, hi = r0 + RP < rows ? r0 + RP : rows;
        while (lo < hi) {
            const int mid = (lo + hi + 1) >> 1;
            if (rowstart[mid] - rowstart[r0] <= static_cast<uint32_t>(cap)) lo = mid;
            else hi = mid - 1;
        }
        const int r1 = lo;
        const bool giant = rowstart[r0 + 1] - rowstart[r0] > static_cast<uint32_t>(cap);
        if (giant) {
            if (t == 0) slow_rows[atomicAdd(slow_count, 1u)] = (static_cast<uint32_t>(b) << 11) | r0;
            r0 = r1;
            continue;
        }
        for (int r = r0 + t; r < r1; r += RP) cursor[r] = rowstart[r] - rowstart[r0];
        __syncthreads();
        if (keep) {
            // from the LDS copy, one run per thread
            for (int q = t; q < nblk; q += RP) {
                const uint32_t* run = ubase + rstart[q];
                const uint32_t len = rstart[q + 1] - rstart[q];
                const uint32_t sbase = static_cast<uint32_t>(q * spb);
                for (uint32_t j = 0; j < len; j += 8) {
                    uint32_t kk[8], pos[8];
#pragma unroll
                    for (int u = 0; u < 8; ++u) kk[u] = j + u < len ? run[j + u] : 0u;
#pragma unroll
                    for (int u = 0; u < 8; ++u) {
                        const int row = static_cast<int>(kk[u] >> hs);
                        pos[u] = (j + u < len && row >= r0 && row < r1) ? atomicAdd(&cursor[row], 1u) : 0xFFFFFFFFu;
                    }
#pragma unroll
                    for (int u = 0; u < 8; ++u)
                        if (pos[u] != 0xFFFFFFFFu)
                            grouped[pos[u]] = (((kk[u] >> sbits) & kmask) << nbits) | (sbase + (kk[u] & smask));
                }
            }
        } else {
            for (int q = t; q < nblk; q += RP) {
                const uint32_t len = rstart[q + 1] - rstart[q];
                const uint32_t* run = part + rbase[q];
                const uint32_t sbase = static_cast<uint32_t>(q * spb);
                for (uint32_t j = 0; j < len; j += kRvGather) {
                    uint32_t kk[kRvGather];
#pragma unroll
                    for (int u = 0; u < kRvGather; ++u) kk[u] = j + u < len ? run[j + u] : 0xFFFFFFFFu;
#pragma unroll
                    for (int u = 0; u < kRvGather; ++u) {
                        if (j + u >= len) continue;
                        const uint32_t key = kk[u];
                        const int row = static_cast<int>(key >> hs);
                        if (row < r0 || row >= r1) continue;
                        grouped[atomicAdd(&cursor[row], 1u)] =
                            (((key >> sbits) & kmask) << nbits) | (sbase + (key & smask));
                    }
                }
            }
        }
        __syncthreads();   // the LDS copy of the keys is dead from here: its space holds the stages
        const int wr0 = r0 + w * 64;
        const int wrn = wr0 < r1 ? (r1 - wr0 < 64 ? r1 - wr0 : 64) : 0;
        rv_stage_in<KMAX>(fwd + (j0 + wr0) * K, wrn, K, wst, lane);
        wave_sync();
        if (lane < wrn) {
            uint32_t* st = wst + lane * ST;
            uint32_t fw[KMAX];
#pragma unroll
            for (int k = 0; k < KMAX; ++k) fw[k] = k < K ? st[k] : 0xFFFFFFFFu;
            const int r = wr0 + lane;
            if (!rv_merge_lane<KMAX>(fw, K, grouped + (rowstart[r] - rowstart[r0]), rowstart[r + 1] - rowstart[r],
                                     nbits, st))
                slow_rows[atomicAdd(slow_count, 1u)] = (static_cast<uint32_t>(b) << 11) | r;
        }
        wave_sync();
        rv_stage_out<KMAX>(out + (j0 + wr0) * K, wrn, K, wst, lane);
        __syncthreads();
        r0 = r1;
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

bool rv_plan(int64_t N, int K, RvPlan& p)
{
    if (N < 1 || K < 1 || K > 64) return false;
    const int64_t E = N * K;
    p.rp = K > 32 ? 128 : 256;
    p.cshift = K > 32 ? 7 : 8;
    while (p.cshift < kRvMaxBinShift && ceil_div(N, int64_t(1) << p.cshift) > kRvMaxBins) ++p.cshift;
    p.nbins = static_cast<int>(ceil_div(N, int64_t(1) << p.cshift));
    if (p.nbins > kRvMaxBins) return false;
    p.nblk = static_cast<int>(std::max<int64_t>(1, std::min<int64_t>(1024, ceil_div(E, 65536))));
    p.spb = ceil_div(ceil_div(N, p.nblk), 4) * 4;
    p.nblk = static_cast<int>(ceil_div(N, p.spb));
    p.kbits = bits_for(K);
    p.sbits = bits_for(p.spb);
    p.nbits = bits_for(N);
    if (p.spb * K >= (int64_t(1) << 24)) return false;           // divmod_small
    if (p.cshift + p.kbits + p.sbits > 32) return false;
    if (p.kbits + p.nbits > 31) return false;   // 0xFFFFFFFF stays free as the empty marker
    if (E >= (int64_t(1) << 32)) return false;
    p.cap = p.rp * K * 17 / 16;
    p.ubuf = std::max(p.cap, p.rp * (K + 1));
    return true;
}

size_t rv_merge_lds(const RvPlan& p, int K)
{
    const size_t words = static_cast<size_t>(2 * p.nblk + 1) + 2 * (size_t(1) << p.cshift) + 1 + p.cap + p.ubuf;
    return words * sizeof(uint32_t);
}

void launch_rv(const uint32_t* fwd, int64_t N, int K, const RvPlan& p, uint32_t* part, uint32_t* meta_cnt,
               uint32_t* meta_off, uint32_t* out, int* err, uint32_t* slow_rows, uint32_t* slow_count, hipStream_t s)
{
#define GT_RV_SCATTER(SC)                                                                                      \
    do {                                                                                                       \
        const size_t lds_s = rv_scatter_lds(p.nbins, SC);                                                      \
        ensure_lds(reinterpret_cast<const void*>(&rv_scatter_kernel<SC>), lds_s);                              \
        hipLaunchKernelGGL((rv_scatter_kernel<SC>), dim3(p.nblk), dim3(kRvScatterThreads), lds_s, s, fwd, N, K,  \
                           p.spb, p.cshift, p.nbins, p.kbits, p.sbits, part, meta_cnt, meta_off, err, slow_count); \
    } while (0)
    if (rv_scatter_lds(p.nbins, 16384) <= 150 * 1024) GT_RV_SCATTER(16384);
    else GT_RV_SCATTER(8192);
#undef GT_RV_SCATTER
    const size_t lds = rv_merge_lds(p, K);
#define GT_RV_MERGE(KM, R)                                                                                       \
    do {                                                                                                         \
        ensure_lds(reinterpret_cast<const void*>(&rv_merge_kernel<KM, R>), lds);                                 \
        hipLaunchKernelGGL((rv_merge_kernel<KM, R>), dim3(p.nbins), dim3(R), lds, s, fwd, N, K, p.nblk, p.spb,   \
                           p.cshift, p.kbits, p.sbits, p.nbits, part, meta_cnt, meta_off, out, p.cap, p.ubuf,    \
                           slow_rows, slow_count);                                                               \
        const size_t lds_w = (2 * static_cast<size_t>(p.nblk) + 1 + 64 * ((KM + 1) / 2) + KM + 1) * 4 * 4;     \
        ensure_lds(reinterpret_cast<const void*>(&rv_slow_kernel<KM>), lds_w);                                   \
        hipLaunchKernelGGL((rv_slow_kernel<KM>), dim3(256), dim3(256), lds_w, s, fwd, N, K, p.nblk, p.spb,       \
                           p.cshift, p.kbits, p.sbits, p.nbits, part, meta_cnt, meta_off, slow_rows, slow_count, \
                           out);                                                                                 \
    } while (0)
    if (K <= 16) GT_RV_MERGE(16, 256);
    else if (K <= 32) GT_RV_MERGE(32, 256);
    else GT_RV_MERGE(64, 128);
#undef GT_RV_MERGE
    GT_HIP(hipGetLastError());
}

}  // namespace gtann
