// refine_kernel.hip -- cross-bucket refinement of neighbour lists (2-hop
// "pull" local join) and the Lloyd centroid update used by bucketing.
//
// Refinement restates src/bucket.cu:4754-4850 (a1_pull_join_kernel): the
// candidates of point a are the first S neighbours of a's first S
// neighbours; invalid ids, a itself and ids already in a's row are dropped,
// duplicates kept once; a candidate survives if its exact distance is
// strictly below a's current M-th distance; the new row is the first M of
// (row U survivors) in (distance, id) order.  Every pass reads the previous
// pass's table (no in-place updates), so the result is deterministic.
#include "gtann_common.hpp"

#include <algorithm>

#include <climits>
#include <cmath>

namespace gtann {

void launch_exclusive_scan(const uint32_t* in, int64_t n, uint32_t* out, uint32_t* sums, hipStream_t s);

constexpr int kRefineMaxCand = 1024;   // S*S
constexpr int kRefineMaxM = 128;
constexpr int kMaxDp = 1024;           // longest padded row of this build

// LDS of one block, sized per launch: the point's row (Dp floats), the id
// hash (H = the power of two >= max(256, 2 (M + S*S)) slots, linear probing
// at load <= 1/2), candidates and their distances (S*S each), survivors and
// theirs (P = the power of two >= S*S each: the bitonic sort pads to it), the
// row and its distances (M each).  At most 37.9 KB (Dp 1024, S*S 1024,
// M 128); 8.9 KB at Dp 96, S 16, M 64, so that the waves, not the LDS,
// limit the blocks per CU (a cap of 2 to 6 blocks per CU measured slower on
// 96- and 960-float rows).
struct RefineLds {
    int H, C, P;
    size_t bytes(int Dp, int M) const { return static_cast<size_t>(Dp + H + 2 * C + 2 * P + 2 * M) * 4; }
};
static RefineLds refine_lds(int M, int S)
{
    RefineLds l{};
    l.C = (S * S + 3) / 4 * 4;
    l.P = 1;
    while (l.P < S * S) l.P <<= 1;
    l.H = 256;
    while (l.H < 2 * (M + S * S)) l.H <<= 1;
    return l;
}

__device__ __forceinline__ bool rkey_less(float da, int32_t ia, float db, int32_t ib)
{
    return da < db || (da == db && ia < ib);
}

// One block per point.  Block b takes position q = (b % 8) * per_xcd + b / 8
// of the processing order (per_xcd = ceil(N / 8)): the workgroups of a
// launch go round-robin to the 8 XCDs, so each XCD walks its own contiguous
// eighth of the order and its L2 keeps the rows of the buckets it is on.
// The order is the last bucketing's member list when there is one (a
// point's 2-hop candidates sit mostly in its own bucket), else the ids.
// The output of a point does not depend on the order.
template <int G>
__global__ void __launch_bounds__(256) refine_2hop_kernel(const float* __restrict__ X, const float* __restrict__ norms,
                                                          int64_t N, int Dp, int metric,
                                                          const int32_t* __restrict__ order,
                                                          const int32_t* __restrict__ in_ids,
                                                          const float* __restrict__ in_d, int M, int S, int H,
                                                          int C, int P, int32_t* __restrict__ out_ids,
                                                          float* __restrict__ out_d)
{
    extern __shared__ __align__(16) float lds[];
    float* xa = lds;                                               // Dp (a multiple of 4)
    int32_t* hkey = reinterpret_cast<int32_t*>(xa + Dp);           // H
    int32_t* cid = hkey + H;                                       // C
    float* cd = reinterpret_cast<float*>(cid + C);                 // C
    int32_t* sid = reinterpret_cast<int32_t*>(cd + C);             // P
    float* sdd = reinterpret_cast<float*>(sid + P);                // P
    int32_t* row = reinterpret_cast<int32_t*>(sdd + P);            // M
    float* rowd = reinterpret_cast<float*>(row + M);               // M
    __shared__ int s_nc, s_ns, s_nr;
    const int64_t per_xcd = (N + 7) / 8;
    const int64_t q = static_cast<int64_t>(blockIdx.x % 8) * per_xcd + blockIdx.x / 8;
    const int tid = threadIdx.x;
    if (q >= N) return;
    const int64_t a = order ? order[q] : q;
    for (int s = tid; s < H; s += 256) hkey[s] = -1;
    for (int k = tid; k < M; k += 256) {
        row[k] = in_ids[a * M + k];
        rowd[k] = in_d[a * M + k];
    }
    for (int d = tid; d < Dp; d += 256) xa[d] = X[a * Dp + d];
    if (tid == 0) { s_nc = 0; s_ns = 0; s_nr = 0; }
    __syncthreads();
    const float kth = rowd[M - 1];
    const float na = metric == 0 ? norms[a] : 0.f;
    const uint32_t mask = static_cast<uint32_t>(H - 1);
    const int hshift = 33 - __ffs(H);   // the top log2(H) bits of the product
    auto insert = [&](int32_t v) -> bool {   // true if v was not present
        uint32_t h = (static_cast<uint32_t>(v) * 2654435761u) >> hshift;
        while (true) {
            const int32_t old = atomicCAS(&hkey[h], -1, v);
            if (old == -1) return true;
            if (old == v) return false;
            h = (h + 1) & mask;
        }
    };
    for (int k = tid; k < M; k += 256) {
        if (row[k] >= 0) {
            insert(row[k]);
            atomicAdd(&s_nr, 1);
        }
    }
    __syncthreads();
    for (int c = tid; c < S * S; c += 256) {
        const int32_t u = row[c / S];
        if (u < 0 || u >= N) continue;
        const int32_t v = in_ids[static_cast<int64_t>(u) * M + (c % S)];
        if (v < 0 || v >= N || v == a) continue;
        if (insert(v)) {
            const int slot = atomicAdd(&s_nc, 1);
            cid[slot] = v;
        }
    }
    __syncthreads();
    const int nc = s_nc;
    // exact distance of every candidate: a group of G lanes per candidate
    // (256 / G candidates in flight per block), lane l of the group reading
    // 16-byte pieces l, l + G, ... of the candidate's row, the point's row
    // broadcast from LDS.  Four partial sums over the dims 4i + c of a lane,
    // (s0 + s1) + (s2 + s3), then a butterfly over the group's lanes.  G = 2
    // for rows of up to 256 floats, 4 beyond (measured on 96- and 960-float
    // rows: one lane per row leaves too few requests per row in flight for
    // long rows, 8 or more lanes too few rows).
    {
        const int g = tid / G, gl = tid % G;
        const int F = Dp / 4;
        const float4* xq = reinterpret_cast<const float4*>(xa);
        for (int k0 = 0; k0 < nc; k0 += 256 / G) {
            const int k = k0 + g;
            float s0 = 0.f, s1 = 0.f, s2 = 0.f, s3 = 0.f;
            if (k < nc) {
                const float4* xv = reinterpret_cast<const float4*>(X + static_cast<int64_t>(cid[k]) * Dp);
                int f = gl;
                // 8 loads in flight before the first use
                for (; f + 7 * G < F; f += 8 * G) {
                    float4 pv[8];
#pragma unroll
                    for (int u = 0; u < 8; ++u) pv[u] = xv[f + u * G];
#pragma unroll
                    for (int u = 0; u < 8; ++u) {
                        const float4 qv = xq[f + u * G];
                        s0 = fmaf(qv.x, pv[u].x, s0);
                        s1 = fmaf(qv.y, pv[u].y, s1);
                        s2 = fmaf(qv.z, pv[u].z, s2);
                        s3 = fmaf(qv.w, pv[u].w, s3);
                    }
                }
                for (; f < F; f += G) {
                    const float4 pv = xv[f];
                    const float4 qv = xq[f];
                    s0 = fmaf(qv.x, pv.x, s0);
                    s1 = fmaf(qv.y, pv.y, s1);
                    s2 = fmaf(qv.z, pv.z, s2);
                    s3 = fmaf(qv.w, pv.w, s3);
                }
            }
            float dot = (s0 + s1) + (s2 + s3);
#pragma unroll
            for (int o = G / 2; o > 0; o >>= 1) dot += __shfl_xor(dot, o);
            if (k < nc && gl == 0) {
                const int32_t v = cid[k];
                cd[k] = metric == 0 ? fmaf(-2.f, dot, norms[v] + na) : -dot;
            }
        }
    }
    __syncthreads();
    // keep d < kth (order fixed later by sorting)
    for (int k = tid; k < nc; k += 256) {
        if (cd[k] < kth) {
            const int slot = atomicAdd(&s_ns, 1);
            sid[slot] = cid[k];
            sdd[slot] = cd[k];
        }
    }
    __syncthreads();
    const int ns = s_ns;
    int n2 = 1;
    while (n2 < ns) n2 <<= 1;
    for (int k = ns + tid; k < n2; k += 256) { sid[k] = INT_MAX; sdd[k] = INFINITY; }
    __syncthreads();
    // bitonic sort of the survivors by (d, id)
    for (int k2 = 2; k2 <= n2; k2 <<= 1) {
        for (int s = k2 >> 1; s > 0; s >>= 1) {
            for (int e = tid; e < n2; e += 256) {
                const int p = e ^ s;
                if (p > e) {
                    const bool asc = (e & k2) == 0;
                    const bool gt = rkey_less(sdd[p], sid[p], sdd[e], sid[e]);
                    if (gt == asc) {
                        const float td = sdd[e]; sdd[e] = sdd[p]; sdd[p] = td;
                        const int32_t ti = sid[e]; sid[e] = sid[p]; sid[p] = ti;
                    }
                }
            }
            __syncthreads();
        }
    }
    const int nr = s_nr;   // valid entries form a prefix of the (sorted) row
    for (int k = tid; k < nr; k += 256) {
        int lo = 0, hi = ns;
        while (lo < hi) {
            const int mid = (lo + hi) >> 1;
            if (rkey_less(sdd[mid], sid[mid], rowd[k], row[k])) lo = mid + 1;
            else hi = mid;
        }
        const int pos = k + lo;
        if (pos < M) { out_ids[a * M + pos] = row[k]; out_d[a * M + pos] = rowd[k]; }
    }
    for (int k = tid; k < ns; k += 256) {
        int lo = 0, hi = nr;
        while (lo < hi) {
            const int mid = (lo + hi) >> 1;
            if (rkey_less(rowd[mid], row[mid], sdd[k], sid[k])) lo = mid + 1;
            else hi = mid;
        }
        const int pos = k + lo;
        if (pos < M) { out_ids[a * M + pos] = sid[k]; out_d[a * M + pos] = sdd[k]; }
    }
    for (int p = nr + ns + tid; p < M; p += 256) { out_ids[a * M + p] = -1; out_d[a * M + p] = INFINITY; }
}

// Lloyd update: centroid c = mean of its member rows; empty buckets keep
// their centroid.  Block (c, h) sums float4 columns [64h, 64h + F) of
// centroid c (F = min(64, Dp / 4 - 64h): up to 256 dimensions per block, so
// long rows spread over several blocks): thread t sums column t % F over its
// group t / F of members (members g, g + G, g + 2G, ... for G = 256 / F
// groups) with four accumulators (members 4k + u of the group into
// accumulator u), folded as (a0 + a1) + (a2 + a3), and the groups are added
// in order.  The result does not depend on scheduling.
__global__ void __launch_bounds__(256) centroid_means_kernel(const float* __restrict__ X, int Dp,
                                                             const int32_t* __restrict__ members,
                                                             const int64_t* __restrict__ off, int64_t C,
                                                             float* __restrict__ cent)
{
    __shared__ float4 part[256];
    const int64_t c = blockIdx.x;
    if (c >= C) return;
    const int64_t lo = off[c], hi = off[c + 1];
    if (hi <= lo) return;
    const int FD = Dp / 4, c0 = static_cast<int>(blockIdx.y) * 64;
    const int F = min(64, FD - c0), G = 256 / F;
    const int col = threadIdx.x % F, g = threadIdx.x / F;
    const float4* X4 = reinterpret_cast<const float4*>(X) + c0 + col;
    float4 a[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) a[u] = make_float4(0.f, 0.f, 0.f, 0.f);
    if (g < G) {
        int64_t i = lo + g;
        for (; i + 3 * G < hi; i += 4 * G) {
            float4 x[4];
#pragma unroll
            for (int u = 0; u < 4; ++u) x[u] = X4[static_cast<int64_t>(members[i + u * G]) * FD];
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                a[u].x += x[u].x; a[u].y += x[u].y; a[u].z += x[u].z; a[u].w += x[u].w;
            }
        }
        for (int u = 0; i < hi; i += G, ++u) {
            const float4 x = X4[static_cast<int64_t>(members[i]) * FD];
            a[u].x += x.x; a[u].y += x.y; a[u].z += x.z; a[u].w += x.w;
        }
    }
    part[threadIdx.x] = make_float4((a[0].x + a[1].x) + (a[2].x + a[3].x), (a[0].y + a[1].y) + (a[2].y + a[3].y),
                                    (a[0].z + a[1].z) + (a[2].z + a[3].z), (a[0].w + a[1].w) + (a[2].w + a[3].w));
    __syncthreads();
    if (threadIdx.x < F) {
        float4 t = make_float4(0.f, 0.f, 0.f, 0.f);
        for (int q = 0; q < G; ++q) {
            const float4 v = part[q * F + threadIdx.x];
            t.x += v.x; t.y += v.y; t.z += v.z; t.w += v.w;
        }
        const float n = static_cast<float>(hi - lo);
        reinterpret_cast<float4*>(cent + c * Dp)[c0 + threadIdx.x] = make_float4(t.x / n, t.y / n, t.z / n, t.w / n);
    }
}

// Stable counting sort on the device (the Lloyd steps' CSR: the sampled
// rows grouped by nearest centroid and, within a centroid, in sample order;
// the bucketing's CSR: two passes, by second key then by bucket) -- the
// order of the host's counting sort.  Each one-wave block owns `chunk`
// consecutive entries: (1) it counts them per key in LDS into
// hist[key][block]; (2) an exclusive scan of hist gives every (key, block)
// pair its output range; (3) it scatters them 64 at a time in input order,
// a lane's rank among the lanes of the same key found by ballots over the
// wave's distinct keys.  out[...] = val[e], or e itself when val is null.
constexpr int kCsrChunk = 256;

__global__ void __launch_bounds__(64) csr_count_kernel(const int32_t* __restrict__ key, int64_t S, int C,
                                                       int64_t chunk, uint32_t* __restrict__ hist)
{
    extern __shared__ uint32_t h[];   // C counters
    const int lane = threadIdx.x;
    for (int i = lane; i < C; i += 64) h[i] = 0u;
    __syncthreads();
    const int64_t e0 = static_cast<int64_t>(blockIdx.x) * chunk, e1 = min(S, e0 + chunk);
    for (int64_t e = e0 + lane; e < e1; e += 64) {
        const int32_t k = key[e];
        if (k >= 0 && k < C) atomicAdd(&h[k], 1u);
    }
    __syncthreads();
    for (int i = lane; i < C; i += 64) hist[static_cast<int64_t>(i) * gridDim.x + blockIdx.x] = h[i];
}

__global__ void __launch_bounds__(64) csr_scatter_kernel(const int32_t* __restrict__ key,
                                                         const int32_t* __restrict__ val, int64_t S, int C,
                                                         int64_t chunk, const uint32_t* __restrict__ offs,
                                                         int32_t* __restrict__ out)
{
    extern __shared__ uint32_t cur[];   // C cursors
    const int lane = threadIdx.x;
    for (int i = lane; i < C; i += 64) cur[i] = offs[static_cast<int64_t>(i) * gridDim.x + blockIdx.x];
    __syncthreads();
    const uint64_t below = lane == 0 ? 0ull : (~0ull >> (64 - lane));
    const int64_t e0 = static_cast<int64_t>(blockIdx.x) * chunk, e1 = min(S, e0 + chunk);
    for (int64_t base = e0; base < e1; base += 64) {
        const int64_t e = base + lane;
        const int32_t k = e < e1 ? key[e] : -1;
        const bool valid = k >= 0 && k < C;
        // the lanes holding the same key as this lane
        uint64_t peers = 0, todo = __ballot(valid);
        while (todo) {
            const int ld = __ffsll(static_cast<unsigned long long>(todo)) - 1;
            const int32_t kl = __shfl(k, ld);
            const uint64_t m = __ballot(valid && k == kl);
            if (valid && k == kl) peers = m;
            todo &= ~m;
        }
        if (valid) out[cur[k] + __popcll(peers & below)] = val ? val[e] : static_cast<int32_t>(e);
        __syncthreads();
        if (valid && (peers >> lane) == 1ull) cur[k] += static_cast<uint32_t>(__popcll(peers));
        __syncthreads();
    }
}

__global__ void csr_offsets_kernel(const uint32_t* __restrict__ offs, int C, int nblk, int64_t* __restrict__ off)
{
    const int c = blockIdx.x * blockDim.x + threadIdx.x;
    if (c <= C) off[c] = offs[static_cast<int64_t>(c) * nblk];
}

void launch_refine_2hop(const float* X, const float* norms, int64_t N, int Dp, int metric, const int32_t* order,
                        const int32_t* in_ids, const float* in_d, int M, int S, int32_t* out_ids, float* out_d,
                        hipStream_t s)
{
    GT_REQUIRE(M <= kRefineMaxM && S * S <= kRefineMaxCand && Dp <= kMaxDp && Dp % 4 == 0,
               "refine limits: M <= 128, S*S <= 1024");
    if (N <= 0) return;
    const dim3 grid(static_cast<unsigned>(8 * ((N + 7) / 8)));
    const int G = Dp <= 256 ? 2 : 4;
    auto k = G == 2 ? refine_2hop_kernel<2> : refine_2hop_kernel<4>;
    const RefineLds l = refine_lds(M, S);
    hipLaunchKernelGGL(k, grid, dim3(256), l.bytes(Dp, M), s, X, norms, N, Dp, metric, order, in_ids, in_d, M, S, l.H, l.C, l.P,
                       out_ids, out_d);
    GT_HIP(hipGetLastError());
}

// entries per block of the stable counting sort: kCsrChunk, more for large
// inputs so that the (key, block) histogram stays near 4,096 blocks
int64_t csr_chunk(int64_t S) { return std::max<int64_t>(kCsrChunk, (S + 4095) / 4096 + 63) / 64 * 64; }
int csr_blocks(int64_t S) { return static_cast<int>((S + csr_chunk(S) - 1) / csr_chunk(S)); }

void launch_sample_csr(const int32_t* key, const int32_t* val, int64_t S, int C, uint32_t* hist, uint32_t* offs,
                       uint32_t* sums, int32_t* members, int64_t* off, hipStream_t s)
{
    GT_REQUIRE(C >= 1 && C <= 16384, "device CSR: at most 16384 keys");
    const int64_t chunk = csr_chunk(S);
    const int nblk = csr_blocks(S);
    const size_t lds = static_cast<size_t>(C) * sizeof(uint32_t);
    if (S > 0) hipLaunchKernelGGL(csr_count_kernel, dim3(nblk), dim3(64), lds, s, key, S, C, chunk, hist);
    launch_exclusive_scan(hist, static_cast<int64_t>(C) * nblk, offs, sums, s);
    if (S > 0)
        hipLaunchKernelGGL(csr_scatter_kernel, dim3(nblk), dim3(64), lds, s, key, val, S, C, chunk, offs, members);
    if (off) hipLaunchKernelGGL(csr_offsets_kernel, dim3((C + 256) / 256), dim3(256), 0, s, offs, C, nblk, off);
    GT_HIP(hipGetLastError());
}

// The bucketing's second key: each point's other top-2 centroid (its own
// bucket when that is missing), key2[i] for the stable sort by (bucket,
// key2, id)
__global__ void bucket_key2_kernel(const uint32_t* __restrict__ top2, const int32_t* __restrict__ bucket, int64_t N,
                                   int64_t C, int32_t* __restrict__ key2)
{
    const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i >= N) return;
    const uint32_t c1 = top2[2 * i], c2 = top2[2 * i + 1];
    const int32_t b = bucket[i];
    const uint32_t other = static_cast<int64_t>(c1) == b ? c2 : c1;
    key2[i] = other < static_cast<uint64_t>(C) ? static_cast<int32_t>(other) : b;
}

// out[i] = min(in[i], 0xFFFF): top-2 centroid lists of fewer than 65,535
// centroids for the host (a missing second centroid stays out of range)
__global__ void pack_u16_kernel(const uint32_t* __restrict__ in, int64_t n, uint16_t* __restrict__ out)
{
    const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i < n) out[i] = static_cast<uint16_t>(min(in[i], 0xFFFFu));
}

void launch_pack_u16(const uint32_t* in, int64_t n, uint16_t* out, hipStream_t s)
{
    if (n <= 0) return;
    hipLaunchKernelGGL(pack_u16_kernel, dim3(static_cast<unsigned>((n + 255) / 256)), dim3(256), 0, s, in, n, out);
    GT_HIP(hipGetLastError());
}

// out[i] = src[idx[i]]
__global__ void gather_i32_kernel(const int32_t* __restrict__ src, const int32_t* __restrict__ idx, int64_t n,
                                  int32_t* __restrict__ out)
{
    const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i < n) out[i] = src[idx[i]];
}

void launch_gather_i32(const int32_t* src, const int32_t* idx, int64_t n, int32_t* out, hipStream_t s)
{
    if (n <= 0) return;
    hipLaunchKernelGGL(gather_i32_kernel, dim3(static_cast<unsigned>((n + 255) / 256)), dim3(256), 0, s, src, idx, n,
                       out);
    GT_HIP(hipGetLastError());
}

// Members of every bucket ordered by (bucket, key2, id) -- the host CSR's
// order -- from the device top-2 lists and the two-choice buckets: key2, a
// stable sort of the ids by key2, their buckets gathered, a stable sort by
// bucket.  members (N) and off (C + 1) out; key2, by_key and bkt (N each)
// and hist / offs / sums (csr_blocks(N) * C, + 1, / 1024 + 2) are scratch.
void launch_bucket_csr(const uint32_t* top2, const int32_t* bucket, int64_t N, int C, int32_t* key2, int32_t* by_key,
                       int32_t* bkt, uint32_t* hist, uint32_t* offs, uint32_t* sums, int32_t* members, int64_t* off,
                       hipStream_t s)
{
    if (N <= 0) return;
    hipLaunchKernelGGL(bucket_key2_kernel, dim3(static_cast<unsigned>((N + 255) / 256)), dim3(256), 0, s, top2, bucket,
                       N, static_cast<int64_t>(C), key2);
    GT_HIP(hipGetLastError());
    launch_sample_csr(key2, nullptr, N, C, hist, offs, sums, by_key, nullptr, s);
    launch_gather_i32(bucket, by_key, N, bkt, s);
    launch_sample_csr(bkt, by_key, N, C, hist, offs, sums, members, off, s);
}

void launch_centroid_sums(const float* X, int Dp, const int32_t* members, const int64_t* offsets, int64_t C,
                          float* centroids, hipStream_t s)
{
    if (C <= 0) return;
    GT_REQUIRE(Dp % 4 == 0, "centroid means: padded rows are multiples of 4 floats");
    const unsigned chunks = static_cast<unsigned>((Dp / 4 + 63) / 64);
    hipLaunchKernelGGL(centroid_means_kernel, dim3(static_cast<unsigned>(C), chunks), dim3(256), 0, s, X, Dp,
                       members, offsets, C, centroids);
    GT_HIP(hipGetLastError());
}

}  // namespace gtann
