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

#include <climits>
#include <cmath>

namespace gtann {

void launch_exclusive_scan(const uint32_t* in, int64_t n, uint32_t* out, uint32_t* sums, hipStream_t s);

constexpr int kRefineMaxCand = 1024;   // S*S
constexpr int kRefineHash = 4096;      // >= 2 * (M + S*S)
constexpr int kRefineMaxM = 128;
constexpr int kMaxDp = 1024;           // longest padded row of this build

__device__ __forceinline__ bool rkey_less(float da, int32_t ia, float db, int32_t ib)
{
    return da < db || (da == db && ia < ib);
}

__global__ void __launch_bounds__(256) refine_2hop_kernel(const float* __restrict__ X, const float* __restrict__ norms,
                                                          int64_t N, int Dp, int metric,
                                                          const int32_t* __restrict__ in_ids,
                                                          const float* __restrict__ in_d, int M, int S,
                                                          int32_t* __restrict__ out_ids, float* __restrict__ out_d)
{
    __shared__ int32_t hkey[kRefineHash];
    __shared__ int32_t cid[kRefineMaxCand];
    __shared__ float cd[kRefineMaxCand];
    __shared__ int32_t row[kRefineMaxM];
    __shared__ float rowd[kRefineMaxM];
    __shared__ float xa[kMaxDp];
    __shared__ int s_nc, s_ns, s_nr;
    const int64_t a = blockIdx.x;
    const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63;
    if (a >= N) return;
    for (int s = tid; s < kRefineHash; s += 256) hkey[s] = -1;
    for (int k = tid; k < M; k += 256) {
        row[k] = in_ids[a * M + k];
        rowd[k] = in_d[a * M + k];
    }
    for (int d = tid; d < Dp; d += 256) xa[d] = X[a * Dp + d];
    if (tid == 0) { s_nc = 0; s_ns = 0; s_nr = 0; }
    __syncthreads();
    const float kth = rowd[M - 1];
    const float na = metric == 0 ? norms[a] : 0.f;
    constexpr uint32_t mask = kRefineHash - 1;
    auto insert = [&](int32_t v) -> bool {   // true if v was not present
        uint32_t h = (static_cast<uint32_t>(v) * 2654435761u) & mask;
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
    // exact distance of every candidate: one wave per candidate, lanes over dims
    for (int k = w; k < nc; k += 4) {
        const int32_t v = cid[k];
        float dot = 0.f;
        for (int d = lane; d < Dp; d += 64) dot = fmaf(xa[d], X[static_cast<int64_t>(v) * Dp + d], dot);
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) dot += __shfl_xor(dot, o);
        if (lane == 0) cd[k] = metric == 0 ? fmaf(-2.f, dot, norms[v] + na) : -dot;
    }
    __syncthreads();
    // keep d < kth, compact in place (order fixed later by sorting)
    __shared__ int32_t sid[kRefineMaxCand];
    __shared__ float sdd[kRefineMaxCand];
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
// their centroid.  One block per centroid.  Dp <= 256 and a multiple of 4:
// thread t sums float4 column t % F (F = Dp / 4) over its group t / F of
// members (members g, g + G, g + 2G, ... for G = 256 / F groups) with four
// accumulators (members 4k + u of the group into accumulator u), folded as
// (a0 + a1) + (a2 + a3), and the groups are added in order.  Other Dp:
// thread t sums dimensions t, t + 256, ... over all members in order.  The
// result does not depend on scheduling.
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
    if (Dp > 256 || Dp % 4 != 0) {
        for (int d = threadIdx.x; d < Dp; d += 256) {
            float t = 0.f;
            for (int64_t i = lo; i < hi; ++i) t += X[static_cast<int64_t>(members[i]) * Dp + d];
            cent[c * Dp + d] = t / static_cast<float>(hi - lo);
        }
        return;
    }
    const int F = Dp / 4, G = 256 / F;
    const int col = threadIdx.x % F, g = threadIdx.x / F;
    const float4* X4 = reinterpret_cast<const float4*>(X);
    float4 a[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) a[u] = make_float4(0.f, 0.f, 0.f, 0.f);
    if (g < G) {
        int64_t i = lo + g;
        for (; i + 3 * G < hi; i += 4 * G) {
            float4 x[4];
#pragma unroll
            for (int u = 0; u < 4; ++u) x[u] = X4[static_cast<int64_t>(members[i + u * G]) * F + col];
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                a[u].x += x[u].x; a[u].y += x[u].y; a[u].z += x[u].z; a[u].w += x[u].w;
            }
        }
        for (int u = 0; i < hi; i += G, ++u) {
            const float4 x = X4[static_cast<int64_t>(members[i]) * F + col];
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
        reinterpret_cast<float4*>(cent + c * Dp)[threadIdx.x] = make_float4(t.x / n, t.y / n, t.z / n, t.w / n);
    }
}

// Lloyd CSR on the device: the sampled rows grouped by nearest centroid and,
// within a centroid, in sample order (a stable counting sort -- the order
// of the host's counting sort).  Each one-wave block owns kCsrChunk
// consecutive sample entries: (1) it counts them per centroid in LDS into
// hist[centroid][block]; (2) an exclusive scan of hist gives every
// (centroid, block) pair its output range; (3) it scatters them 64 at a
// time in sample order, a lane's rank among the lanes of the same centroid
// found by ballots over the wave's distinct keys.
constexpr int kCsrChunk = 1024;

__global__ void __launch_bounds__(64) csr_count_kernel(const int32_t* __restrict__ key, int64_t S, int C,
                                                       uint32_t* __restrict__ hist)
{
    extern __shared__ uint32_t h[];   // C counters
    const int lane = threadIdx.x;
    for (int i = lane; i < C; i += 64) h[i] = 0u;
    __syncthreads();
    const int64_t e0 = static_cast<int64_t>(blockIdx.x) * kCsrChunk, e1 = min(S, e0 + kCsrChunk);
    for (int64_t e = e0 + lane; e < e1; e += 64) {
        const int32_t k = key[e];
        if (k >= 0 && k < C) atomicAdd(&h[k], 1u);
    }
    __syncthreads();
    for (int i = lane; i < C; i += 64) hist[static_cast<int64_t>(i) * gridDim.x + blockIdx.x] = h[i];
}

__global__ void __launch_bounds__(64) csr_scatter_kernel(const int32_t* __restrict__ key,
                                                         const int32_t* __restrict__ val, int64_t S, int C,
                                                         const uint32_t* __restrict__ offs, int32_t* __restrict__ out)
{
    extern __shared__ uint32_t cur[];   // C cursors
    const int lane = threadIdx.x;
    for (int i = lane; i < C; i += 64) cur[i] = offs[static_cast<int64_t>(i) * gridDim.x + blockIdx.x];
    __syncthreads();
    const uint64_t below = lane == 0 ? 0ull : (~0ull >> (64 - lane));
    const int64_t e0 = static_cast<int64_t>(blockIdx.x) * kCsrChunk, e1 = min(S, e0 + kCsrChunk);
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
        if (valid) out[cur[k] + __popcll(peers & below)] = val[e];
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

void launch_refine_2hop(const float* X, const float* norms, int64_t N, int Dp, int metric, const int32_t* in_ids,
                        const float* in_d, int M, int S, int32_t* out_ids, float* out_d, hipStream_t s)
{
    GT_REQUIRE(M <= kRefineMaxM && S * S <= kRefineMaxCand && Dp <= kMaxDp, "refine limits: M <= 128, S*S <= 1024");
    if (N <= 0) return;
    hipLaunchKernelGGL(refine_2hop_kernel, dim3(static_cast<unsigned>(N)), dim3(256), 0, s, X, norms, N, Dp, metric,
                       in_ids, in_d, M, S, out_ids, out_d);
    GT_HIP(hipGetLastError());
}

int csr_blocks(int64_t S) { return static_cast<int>((S + kCsrChunk - 1) / kCsrChunk); }

void launch_sample_csr(const int32_t* key, const int32_t* val, int64_t S, int C, uint32_t* hist, uint32_t* offs,
                       uint32_t* sums, int32_t* members, int64_t* off, hipStream_t s)
{
    GT_REQUIRE(C >= 1 && C <= 16384, "device CSR: at most 16384 keys");
    const int nblk = csr_blocks(S);
    const size_t lds = static_cast<size_t>(C) * sizeof(uint32_t);
    if (S > 0) hipLaunchKernelGGL(csr_count_kernel, dim3(nblk), dim3(64), lds, s, key, S, C, hist);
    launch_exclusive_scan(hist, static_cast<int64_t>(C) * nblk, offs, sums, s);
    if (S > 0) hipLaunchKernelGGL(csr_scatter_kernel, dim3(nblk), dim3(64), lds, s, key, val, S, C, offs, members);
    hipLaunchKernelGGL(csr_offsets_kernel, dim3((C + 256) / 256), dim3(256), 0, s, offs, C, nblk, off);
    GT_HIP(hipGetLastError());
}

void launch_centroid_sums(const float* X, int Dp, const int32_t* members, const int64_t* offsets, int64_t C,
                          float* centroids, hipStream_t s)
{
    if (C <= 0) return;
    hipLaunchKernelGGL(centroid_means_kernel, dim3(static_cast<unsigned>(C)), dim3(256), 0, s, X, Dp, members,
                       offsets, C, centroids);
    GT_HIP(hipGetLastError());
}

}  // namespace gtann
