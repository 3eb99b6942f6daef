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
// their centroid.  One block per centroid.  Dp <= 256: thread t sums
// dimension t % Dp over members t / Dp, t / Dp + parts, ... and the parts are
// added in a fixed order; Dp > 256: thread t sums dimensions t, t + 256, ...
// over all members in order.  The result does not depend on scheduling.
__global__ void __launch_bounds__(256) centroid_means_kernel(const float* __restrict__ X, int Dp,
                                                             const int32_t* __restrict__ members,
                                                             const int64_t* __restrict__ off, int64_t C,
                                                             float* __restrict__ cent)
{
    __shared__ float part[256];
    const int64_t c = blockIdx.x;
    if (c >= C) return;
    const int64_t lo = off[c], hi = off[c + 1];
    if (hi <= lo) return;
    if (Dp > 256) {
        for (int d = threadIdx.x; d < Dp; d += 256) {
            float t = 0.f;
            for (int64_t i = lo; i < hi; ++i) t += X[static_cast<int64_t>(members[i]) * Dp + d];
            cent[c * Dp + d] = t / static_cast<float>(hi - lo);
        }
        return;
    }
    const int parts = Dp <= 256 ? 256 / Dp : 1;
    const int d = threadIdx.x % Dp, pidx = threadIdx.x / Dp;
    float s = 0.f;
    if (pidx < parts) {
        int64_t i = lo + pidx;
        for (; i + 3 * parts < hi; i += 4 * parts) {
            const float a0 = X[static_cast<int64_t>(members[i]) * Dp + d];
            const float a1 = X[static_cast<int64_t>(members[i + parts]) * Dp + d];
            const float a2 = X[static_cast<int64_t>(members[i + 2 * parts]) * Dp + d];
            const float a3 = X[static_cast<int64_t>(members[i + 3 * parts]) * Dp + d];
            s += (a0 + a1) + (a2 + a3);
        }
        for (; i < hi; i += parts) s += X[static_cast<int64_t>(members[i]) * Dp + d];
    }
    part[threadIdx.x] = s;
    __syncthreads();
    if (threadIdx.x < Dp) {
        float t = 0.f;
        for (int p = 0; p < parts; ++p) t += part[p * Dp + threadIdx.x];
        cent[c * Dp + threadIdx.x] = t / static_cast<float>(hi - lo);
    }
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

void launch_centroid_sums(const float* X, int Dp, const int32_t* members, const int64_t* offsets, int64_t C,
                          float* centroids, hipStream_t s)
{
    if (C <= 0) return;
    hipLaunchKernelGGL(centroid_means_kernel, dim3(static_cast<unsigned>(C)), dim3(256), 0, s, X, Dp, members,
                       offsets, C, centroids);
    GT_HIP(hipGetLastError());
}

}  // namespace gtann
