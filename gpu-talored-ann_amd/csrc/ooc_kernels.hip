// ooc_kernels.hip -- kernels of the out-of-core path: stages that hold only
// a chunk of the N x M / N x K tables on the device at a time (the host keeps
// the rest), for graphs whose tables exceed a device memory budget
// (src/bucket.cu:5670-6369 ChunkedKnnAccumulator, src/prune_windowed_gpu.cu:
// 529-915 run_chunked, src/optimize_chunked.cu:1548-2057 multi-chunk Method E).
#include "gtann_common.hpp"

namespace gtann {

// cidx[ids[i]] = i: the compact row of every id a prune chunk reads.  Entries
// of ids not in the list keep whatever an earlier chunk wrote; the chunk reads
// only listed ids.
__global__ void set_cidx_kernel(const int32_t* __restrict__ ids, int64_t n, int32_t* __restrict__ cidx)
{
    const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i < n) cidx[ids[i]] = static_cast<int32_t>(i);
}

// Reverse edges of a batch of forward rows (rows s0 .. s0 + nrows - 1 of an
// N x K graph), routed to destination chunks of R consecutive rows.  A
// record is (rank << 58) | (dst - chunk * R) << 32 | src.  Pass 1 counts the
// records per chunk (LDS counters, one global add per block and chunk);
// pass 2 places them at the chunk's cursor in the batch buffer.
constexpr int kRouteThreads = 256;
constexpr int kRouteMaxChunks = 4096;

__global__ void __launch_bounds__(kRouteThreads) route_count_kernel(const uint32_t* __restrict__ fwd, int64_t nrows,
                                                                    int K, int64_t N, int64_t R, int nchunks,
                                                                    uint32_t* __restrict__ counts,
                                                                    int* __restrict__ err)
{
    __shared__ uint32_t cnt[kRouteMaxChunks];
    for (int c = threadIdx.x; c < nchunks; c += kRouteThreads) cnt[c] = 0u;
    __syncthreads();
    const int64_t E = nrows * K;
    bool bad = false;
    for (int64_t e = static_cast<int64_t>(blockIdx.x) * kRouteThreads + threadIdx.x; e < E;
         e += static_cast<int64_t>(gridDim.x) * kRouteThreads) {
        const uint32_t j = fwd[e];
        if (j >= N) bad = true;
        else atomicAdd(&cnt[j / R], 1u);
    }
    if (bad) atomicExch(err, 1);
    __syncthreads();
    for (int c = threadIdx.x; c < nchunks; c += kRouteThreads)
        if (cnt[c]) atomicAdd(&counts[c], cnt[c]);
}

__global__ void __launch_bounds__(kRouteThreads) route_place_kernel(const uint32_t* __restrict__ fwd, int64_t nrows,
                                                                    int K, int64_t N, int64_t R, int64_t s0,
                                                                    uint32_t* __restrict__ cursor,
                                                                    unsigned long long* __restrict__ recs)
{
    const int64_t E = nrows * K;
    for (int64_t e = static_cast<int64_t>(blockIdx.x) * kRouteThreads + threadIdx.x; e < E;
         e += static_cast<int64_t>(gridDim.x) * kRouteThreads) {
        const uint32_t j = fwd[e];
        if (j >= N) continue;
        const int64_t i = e / K;
        const uint64_t k = static_cast<uint64_t>(e - i * K);
        const uint64_t c = j / R;
        const uint64_t dl = j - c * R;
        recs[atomicAdd(&cursor[c], 1u)] = (k << 58) | (dl << 32) | static_cast<uint32_t>(s0 + i);
    }
}

// A destination chunk's records grouped per row (CSR, the key order inside a
// row is free): deg / slot by atomics, then keys (rank << 32 | src) at
// off[row] + slot -- the layout rev_merge_kernel reads.
__global__ void rec_count_kernel(const unsigned long long* __restrict__ recs, int64_t n, uint32_t* __restrict__ deg,
                                 uint32_t* __restrict__ slot)
{
    const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const uint32_t dl = static_cast<uint32_t>((recs[i] >> 32) & 0x3FFFFFFull);
    slot[i] = atomicAdd(&deg[dl], 1u);
}

__global__ void rec_scatter_kernel(const unsigned long long* __restrict__ recs, int64_t n,
                                   const uint32_t* __restrict__ off, const uint32_t* __restrict__ slot,
                                   unsigned long long* __restrict__ keys)
{
    const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const unsigned long long r = recs[i];
    const uint32_t dl = static_cast<uint32_t>((r >> 32) & 0x3FFFFFFull);
    keys[off[dl] + slot[i]] = ((r >> 58) << 32) | static_cast<uint32_t>(r);
}

static unsigned grid_of(int64_t n, int b) { return static_cast<unsigned>(std::max<int64_t>(1, ceil_div(n, b))); }

void launch_set_cidx(const int32_t* ids, int64_t n, int32_t* cidx, hipStream_t s)
{
    if (n <= 0) return;
    hipLaunchKernelGGL(set_cidx_kernel, dim3(grid_of(n, 256)), dim3(256), 0, s, ids, n, cidx);
    GT_HIP(hipGetLastError());
}

void launch_route(const uint32_t* fwd, int64_t nrows, int K, int64_t N, int64_t R, int nchunks, int64_t s0,
                  uint32_t* counts, uint32_t* cursor, unsigned long long* recs, int* err, bool place, hipStream_t s)
{
    GT_REQUIRE(nchunks >= 1 && nchunks <= kRouteMaxChunks, "too many destination chunks");
    GT_REQUIRE(R <= (int64_t(1) << 26) && K <= 64, "destination chunk or degree too large for a route record");
    if (nrows <= 0) return;
    const unsigned grid = static_cast<unsigned>(std::min<int64_t>(2048, ceil_div(nrows * K, kRouteThreads)));
    if (!place)
        hipLaunchKernelGGL(route_count_kernel, dim3(grid), dim3(kRouteThreads), 0, s, fwd, nrows, K, N, R, nchunks,
                           counts, err);
    else
        hipLaunchKernelGGL(route_place_kernel, dim3(grid), dim3(kRouteThreads), 0, s, fwd, nrows, K, N, R, s0, cursor,
                           recs);
    GT_HIP(hipGetLastError());
}

void launch_rec_group(const unsigned long long* recs, int64_t n, uint32_t* deg, uint32_t* slot, const uint32_t* off,
                      unsigned long long* keys, bool scatter, hipStream_t s)
{
    if (n <= 0) return;
    if (!scatter)
        hipLaunchKernelGGL(rec_count_kernel, dim3(grid_of(n, 256)), dim3(256), 0, s, recs, n, deg, slot);
    else
        hipLaunchKernelGGL(rec_scatter_kernel, dim3(grid_of(n, 256)), dim3(256), 0, s, recs, n, off, slot, keys);
    GT_HIP(hipGetLastError());
}

}  // namespace gtann
