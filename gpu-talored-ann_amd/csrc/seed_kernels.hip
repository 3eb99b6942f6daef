// seed_kernels.hip -- KMeans|| (scalable k-means++, Bahmani et al. 2012)
// oversampling of the bucketing's centroid seeds on the device, the
// algorithm of src/bucket.cu:2833-3168: the squared distance of every
// training row to its nearest candidate is kept in HBM, each round samples
// rows independently with probability l*k*d^2/psi (psi estimated from every
// stride-th row, src/bucket.cu:3003-3016), and the new candidates lower the
// distances.  The distances to new candidates come from the fused MFMA kNN
// kernel with lists of one (gtann_api.hip); these kernels are the
// elementwise steps around it.
#include "gtann_common.hpp"

#include <algorithm>

namespace gtann {

// splitmix64's output function: a counter-based uniform draw per (seed, row)
__device__ inline uint64_t seed_mix64(uint64_t z)
{
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

// flag[i] = (i == first) (row `first` is the first candidate), mind[i] = +inf
__global__ void kmpar_init_kernel(uint8_t* __restrict__ flag, float* __restrict__ mind, int64_t S, int64_t first)
{
    const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i >= S) return;
    flag[i] = i == first ? 1 : 0;
    mind[i] = __builtin_inff();
}

// psi = scale * sum of mind[0], mind[stride], ..., mind[(nsub - 1) * stride]
// (one block; the sum in double)
__global__ void __launch_bounds__(1024) kmpar_psi_kernel(const float* __restrict__ mind, int64_t stride, int64_t nsub,
                                                         double scale, float* __restrict__ psi)
{
    __shared__ double part[1024 / 64];
    double s = 0.0;
    for (int64_t k = threadIdx.x; k < nsub; k += blockDim.x) s += static_cast<double>(fmaxf(mind[k * stride], 0.f));
    for (int o = 32; o >= 1; o >>= 1) s += __shfl_xor(s, o);
    const int w = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 0) part[w] = s;
    __syncthreads();
    if (threadIdx.x == 0) {
        double t = 0.0;
        for (int k = 0; k < static_cast<int>(blockDim.x >> 6); ++k) t += part[k];
        *psi = static_cast<float>(t * scale);
    }
}

// D^2 sampling: row i (not yet a candidate) is taken when its uniform draw
// is below lk * d^2(i) / psi (src/bucket.cu:2548-2561); sel[i] = taken
__global__ void kmpar_sample_kernel(const float* __restrict__ mind, uint8_t* __restrict__ flag,
                                    uint32_t* __restrict__ sel, int64_t S, const float* __restrict__ psi, float lk,
                                    uint64_t seed)
{
    const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i >= S) return;
    const float ps = *psi;
    const float u = static_cast<float>(seed_mix64(seed + static_cast<uint64_t>(i) * 0x9E3779B97F4A7C15ull) >> 40) *
                    (1.0f / 16777216.0f);
    const bool take = !flag[i] && ps > 0.f && u * ps < lk * fmaxf(mind[i], 0.f);
    sel[i] = take ? 1u : 0u;
    if (take) flag[i] = 1;
}

// out[pos[i]] = rows[i] for every selected row, in row order
__global__ void kmpar_compact_kernel(const uint32_t* __restrict__ sel, const uint32_t* __restrict__ pos,
                                     const int32_t* __restrict__ rows, int64_t S, int32_t* __restrict__ out)
{
    const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i >= S || !sel[i]) return;
    out[pos[i]] = rows[i];
}

// mind = min(mind, dnew), distances below 0 (fp32 rounding of an expanded
// form) taken as 0
__global__ void kmpar_min_kernel(float* __restrict__ mind, const float* __restrict__ dnew, int64_t S)
{
    const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i >= S) return;
    mind[i] = fminf(mind[i], fmaxf(dnew[i], 0.f));
}

// out row k = X row ids[k] (Dp floats per row, 16-byte words)
__global__ void gather_rows_f32_kernel(const float4* __restrict__ X, int w4, const int32_t* __restrict__ ids,
                                       int64_t n, float4* __restrict__ out)
{
    const int64_t e = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (e >= n * w4) return;
    const int64_t k = e / w4;
    const int c = static_cast<int>(e - k * w4);
    out[e] = X[static_cast<int64_t>(ids[k]) * w4 + c];
}

static unsigned grid256(int64_t n) { return static_cast<unsigned>((n + 255) / 256); }

void launch_kmpar_init(uint8_t* flag, float* mind, int64_t S, int64_t first, hipStream_t s)
{
    if (S <= 0) return;
    hipLaunchKernelGGL(kmpar_init_kernel, dim3(grid256(S)), dim3(256), 0, s, flag, mind, S, first);
    GT_HIP(hipGetLastError());
}

void launch_kmpar_psi(const float* mind, int64_t S, int64_t target, float* psi, hipStream_t s)
{
    const int64_t stride = std::max<int64_t>(1, S / std::max<int64_t>(1, target));
    const int64_t nsub = std::max<int64_t>(1, S / stride);
    hipLaunchKernelGGL(kmpar_psi_kernel, dim3(1), dim3(1024), 0, s, mind, stride, nsub,
                       static_cast<double>(S) / static_cast<double>(nsub), psi);
    GT_HIP(hipGetLastError());
}

void launch_kmpar_sample(const float* mind, uint8_t* flag, uint32_t* sel, int64_t S, const float* psi, float lk,
                         uint64_t seed, hipStream_t s)
{
    if (S <= 0) return;
    hipLaunchKernelGGL(kmpar_sample_kernel, dim3(grid256(S)), dim3(256), 0, s, mind, flag, sel, S, psi, lk, seed);
    GT_HIP(hipGetLastError());
}

void launch_kmpar_compact(const uint32_t* sel, const uint32_t* pos, const int32_t* rows, int64_t S, int32_t* out,
                          hipStream_t s)
{
    if (S <= 0) return;
    hipLaunchKernelGGL(kmpar_compact_kernel, dim3(grid256(S)), dim3(256), 0, s, sel, pos, rows, S, out);
    GT_HIP(hipGetLastError());
}

void launch_kmpar_min(float* mind, const float* dnew, int64_t S, hipStream_t s)
{
    if (S <= 0) return;
    hipLaunchKernelGGL(kmpar_min_kernel, dim3(grid256(S)), dim3(256), 0, s, mind, dnew, S);
    GT_HIP(hipGetLastError());
}

void launch_gather_rows_f32(const float* X, int Dp, const int32_t* ids, int64_t n, float* out, hipStream_t s)
{
    GT_REQUIRE(Dp % 4 == 0, "gather_rows_f32: padded dimension must be a multiple of 4");
    if (n <= 0) return;
    const int w4 = Dp / 4;
    hipLaunchKernelGGL(gather_rows_f32_kernel, dim3(grid256(n * w4)), dim3(256), 0, s,
                       reinterpret_cast<const float4*>(X), w4, ids, n, reinterpret_cast<float4*>(out));
    GT_HIP(hipGetLastError());
}

}  // namespace gtann
