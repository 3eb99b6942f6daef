// occlusion_kernels.hip -- the two neighbour-list stages of the Python
// pipeline on gfx950:
//
//   * occlusion prune of bd/prune.py:8-83 (prune_graph): per point v the
//     valid candidates (not -1, not out of range, not v) are ordered by
//     d(v, z); walking that order, z is dropped when an earlier kept u has
//     d(u, z) < d(v, z); the kept ids, truncated to max_degree, are written
//     left-aligned and the rest of the row is -1;
//   * reverse-edge insertion of bd/build_bucket.py:473-543
//     (_apply_reverse_edges): every forward edge a -> b with distance d is
//     offered to b's list; b's new list is the M smallest of its current list
//     and the offered sources that are not already in it.
//
// Occlusion prune: one wave per point.  The pairwise distances among the M
// candidates come from their Gram matrix on the fp32 matrix cores
// (d(u,z) = |u|^2 + |z|^2 - 2 u.z); the candidate rows are read straight
// from HBM into MFMA operand registers, half of the dimensions per half-wave.
// The greedy walk then works on one 128-bit "occluded by" mask per candidate
// (bit r set = the candidate of rank r occludes it), so the sequential part
// is a scalar loop of a few instructions per candidate.
#include "gtann_common.hpp"

#include <climits>
#include <cmath>

namespace gtann {

typedef float floatx16 __attribute__((ext_vector_type(16)));

constexpr int kOccMaxM = 128;

__device__ __forceinline__ uint64_t readlane_u64(uint64_t v, int l)
{
    const uint32_t lo = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(v), l));
    const uint32_t hi = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(v >> 32), l));
    return (static_cast<uint64_t>(hi) << 32) | lo;
}

// NB = candidate blocks of 32 (M <= 32*NB); CG = Gram tile columns per pass
// (the accumulators of one pass are NB*CG 32x32 tiles).
template <int NB, int CG>
__global__ void __launch_bounds__(256) occlusion_prune_kernel(const float* __restrict__ X, int64_t N, int Dp,
                                                              const int32_t* __restrict__ nb, int M, int max_deg,
                                                              int32_t* __restrict__ out)
{
    constexpr int MC = NB * 32;
    __shared__ int32_t s_id[4][MC];
    __shared__ float s_n[4][MC];
    __shared__ float s_dv[4][MC];
    __shared__ int32_t s_rank[4][MC];
    __shared__ int32_t s_ord[4][MC];
    __shared__ uint64_t s_cm[4][MC][2];
    const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int64_t v = static_cast<int64_t>(blockIdx.x) * 4 + w;
    if (v >= N) return;   // the whole wave leaves; only wave-level syncs below
    const int half = lane >> 5, r32 = lane & 31;
    const int DH = Dp >> 1;

    for (int c = lane; c < MC; c += 64) {
        int32_t z = c < M ? nb[v * M + c] : -1;
        if (z < 0 || z >= N || z == v) z = -1;
        s_id[w][c] = z;
    }
    wave_sync();

    // lane (half, r32) streams dims [half*DH, half*DH + DH) of candidate
    // I*32 + r32 for every block I; invalid candidates read v's row, zeroed
    const float* rp[NB];
    bool rv[NB];
#pragma unroll
    for (int I = 0; I < NB; ++I) {
        const int32_t z = s_id[w][I * 32 + r32];
        rv[I] = z >= 0;
        rp[I] = X + (rv[I] ? static_cast<int64_t>(z) : v) * Dp + half * DH;
    }
    const float* vp = X + v * Dp + half * DH;
    float nrm[NB], dvp[NB];
#pragma unroll
    for (int I = 0; I < NB; ++I) { nrm[I] = 0.f; dvp[I] = 0.f; }

#pragma unroll
    for (int J0 = 0; J0 < NB; J0 += CG) {
        floatx16 acc[NB][CG];
#pragma unroll
        for (int I = 0; I < NB; ++I)
#pragma unroll
            for (int c = 0; c < CG; ++c)
#pragma unroll
                for (int r = 0; r < 16; ++r) acc[I][c][r] = 0.f;

        for (int d0 = 0; d0 < DH; d0 += 8) {
            float a[NB][8];
#pragma unroll
            for (int I = 0; I < NB; ++I) {
                const float4 x0 = *reinterpret_cast<const float4*>(rp[I] + d0);
                const float4 x1 = *reinterpret_cast<const float4*>(rp[I] + d0 + 4);
                const float m = rv[I] ? 1.f : 0.f;
                a[I][0] = x0.x * m; a[I][1] = x0.y * m; a[I][2] = x0.z * m; a[I][3] = x0.w * m;
                a[I][4] = x1.x * m; a[I][5] = x1.y * m; a[I][6] = x1.z * m; a[I][7] = x1.w * m;
            }
            if (J0 == 0) {
                const float4 v0 = *reinterpret_cast<const float4*>(vp + d0);
                const float4 v1 = *reinterpret_cast<const float4*>(vp + d0 + 4);
                const float vv[8] = {v0.x, v0.y, v0.z, v0.w, v1.x, v1.y, v1.z, v1.w};
#pragma unroll
                for (int I = 0; I < NB; ++I)
#pragma unroll
                    for (int e = 0; e < 8; ++e) {
                        nrm[I] = fmaf(a[I][e], a[I][e], nrm[I]);
                        const float t = a[I][e] - vv[e];
                        dvp[I] = fmaf(t, t, dvp[I]);
                    }
            }
#pragma unroll
            for (int s = 0; s < 8; ++s)
#pragma unroll
                for (int I = 0; I < NB; ++I)
#pragma unroll
                    for (int c = 0; c < CG; ++c)
                        if (J0 + c < NB)
                            acc[I][c] = __builtin_amdgcn_mfma_f32_32x32x2f32(a[I][s], a[J0 + c][s], acc[I][c], 0, 0, 0);
        }

        if (J0 == 0) {
            // |z|^2 and d(v, z) of every candidate, then its rank in
            // (d(v, z), position) order; invalid candidates rank last
#pragma unroll
            for (int I = 0; I < NB; ++I) {
                nrm[I] += __shfl_xor(nrm[I], 32);
                dvp[I] += __shfl_xor(dvp[I], 32);
                if (half == 0) {
                    s_n[w][I * 32 + r32] = nrm[I];
                    s_dv[w][I * 32 + r32] = rv[I] ? dvp[I] : INFINITY;
                }
            }
            wave_sync();
            for (int c = lane; c < MC; c += 64) {
                auto okey = [&](int x) -> uint64_t {
                    const uint32_t hi = s_id[w][x] >= 0 ? f2o(s_dv[w][x]) : 0xFFFFFFFFu;
                    return (static_cast<uint64_t>(hi) << 32) | static_cast<uint32_t>(x);
                };
                const uint64_t kc = okey(c);
                int rk = 0;
                for (int x = 0; x < MC; ++x) rk += okey(x) < kc ? 1 : 0;
                s_rank[w][c] = rk;
                s_ord[w][rk] = c;
            }
            wave_sync();
        }

        // occlusion masks of the columns of this pass, indexed by rank
#pragma unroll
        for (int c = 0; c < CG; ++c) {
            const int J = J0 + c;
            if (J >= NB) continue;
            const int j = J * 32 + r32;
            const int32_t idj = s_id[w][j];
            const int rj = s_rank[w][j];
            const float dvj = s_dv[w][j], nj = s_n[w][j];
            uint64_t lo = 0, hi = 0;
#pragma unroll
            for (int I = 0; I < NB; ++I)
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int i = I * 32 + 8 * (r >> 2) + 4 * half + (r & 3);
                    const int32_t idi = s_id[w][i];
                    const int ri = s_rank[w][i];
                    const float d = idi == idj ? 0.f : fmaf(-2.f, acc[I][c][r], s_n[w][i] + nj);
                    if (idi >= 0 && idj >= 0 && ri < rj && d < dvj) {
                        if (ri < 64) lo |= 1ull << ri;
                        else hi |= 1ull << (ri - 64);
                    }
                }
            lo |= shfl_xor_u64(lo, 32);
            hi |= shfl_xor_u64(hi, 32);
            if (half == 0 && idj >= 0) {
                s_cm[w][rj][0] = lo;
                s_cm[w][rj][1] = hi;
            }
        }
    }
    wave_sync();

    // greedy walk in rank order over the valid candidates
    int cnt = __popcll(__ballot(lane < MC && s_id[w][lane < MC ? lane : 0] >= 0));
    if (MC > 64) cnt += __popcll(__ballot(lane + 64 < MC && s_id[w][lane + 64 < MC ? lane + 64 : 0] >= 0));
    uint64_t m0lo = 0, m0hi = 0, m1lo = 0, m1hi = 0;
    if (lane < cnt) { m0lo = s_cm[w][lane][0]; m0hi = s_cm[w][lane][1]; }
    if (MC > 64 && lane + 64 < cnt) { m1lo = s_cm[w][lane + 64][0]; m1hi = s_cm[w][lane + 64][1]; }
    const int limit = max_deg > 0 ? max_deg : INT_MAX;
    uint64_t klo = 0, khi = 0;
    int kept = 0;
    for (int p = 0; p < cnt && kept < limit; ++p) {
        uint64_t lo, hi;
        if (p < 64) {
            lo = readlane_u64(m0lo, p);
            hi = readlane_u64(m0hi, p);
        } else {
            lo = readlane_u64(m1lo, p - 64);
            hi = readlane_u64(m1hi, p - 64);
        }
        if (((lo & klo) | (hi & khi)) == 0) {
            if (p < 64) klo |= 1ull << p;
            else khi |= 1ull << (p - 64);
            ++kept;
        }
    }
    for (int p = lane; p < MC; p += 64) {
        const bool k = p < 64 ? ((klo >> p) & 1) : ((khi >> (p - 64)) & 1);
        if (!k) continue;
        const int slot = p < 64 ? __popcll(klo & ((1ull << p) - 1))
                                : __popcll(klo) + __popcll(khi & ((1ull << (p - 64)) - 1));
        out[v * M + slot] = s_id[w][s_ord[w][p]];
    }
    for (int s = kept + lane; s < M; s += 64) out[v * M + s] = -1;
}

// ------------------------------------------------------ reverse-edge insertion

constexpr int kRinMaxM = 128;
constexpr int kRinHash = 256;   // open addressing, >= 2 * M

__global__ void rin_worst_kernel(const float* __restrict__ d, int64_t N, int M, float* __restrict__ worst)
{
    const int64_t b = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (b >= N) return;
    float w = -INFINITY;
    for (int k = 0; k < M; ++k) w = fmaxf(w, d[b * M + k]);
    worst[b] = w;
}

// A forward edge a -> b is offered to b only if its distance is strictly
// below b's current worst; each kept edge takes the next slot of b's segment.
__global__ void rin_count_kernel(const int32_t* __restrict__ ids, const float* __restrict__ d, int64_t E, int64_t N,
                                 const float* __restrict__ worst, uint32_t* __restrict__ cnt,
                                 uint32_t* __restrict__ slot, int* __restrict__ err)
{
    const int64_t e = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (e >= E) return;
    const int32_t b = ids[e];
    uint32_t s = ~0u;
    if (b >= N) atomicExch(err, 1);
    else if (b >= 0 && d[e] < worst[b]) s = atomicAdd(&cnt[b], 1u);
    slot[e] = s;
}

__global__ void rin_scatter_kernel(const int32_t* __restrict__ ids, const float* __restrict__ d, int64_t E, int M,
                                   const uint32_t* __restrict__ off, const uint32_t* __restrict__ slot,
                                   unsigned long long* __restrict__ keys)
{
    const int64_t e = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (e >= E) return;
    const uint32_t s = slot[e];
    if (s == ~0u) return;
    keys[off[ids[e]] + s] = pack_key(d[e], static_cast<int32_t>(e / M));
}

__device__ __forceinline__ uint64_t wave_sort64_u64(uint64_t x, int lane)
{
#pragma unroll
    for (int k = 2; k <= 64; k <<= 1)
#pragma unroll
        for (int j = k >> 1; j > 0; j >>= 1) {
            const uint64_t o = shfl_xor_u64(x, j);
            const bool asc = (lane & k) == 0, lower = (lane & j) == 0;
            x = (lower == asc) ? (x < o ? x : o) : (x < o ? o : x);
        }
    return x;
}

// ascending sort of 128 keys held as (e0 at index lane, e1 at index lane + 64)
__device__ __forceinline__ void wave_sort128_u64(uint64_t& e0, uint64_t& e1, int lane)
{
#pragma unroll
    for (int k = 2; k <= 128; k <<= 1)
#pragma unroll
        for (int j = k >> 1; j > 0; j >>= 1) {
            if (j == 64) {
                const uint64_t lo = e0 < e1 ? e0 : e1, hi = e0 < e1 ? e1 : e0;
                e0 = lo;
                e1 = hi;
                continue;
            }
            const uint64_t o0 = shfl_xor_u64(e0, j), o1 = shfl_xor_u64(e1, j);
            const bool lower = (lane & j) == 0;
            const bool asc0 = (lane & k) == 0, asc1 = ((lane + 64) & k) == 0;
            e0 = (lower == asc0) ? (e0 < o0 ? e0 : o0) : (e0 < o0 ? o0 : e0);
            e1 = (lower == asc1) ? (e1 < o1 ? e1 : o1) : (e1 < o1 ? o1 : e1);
        }
}

// One wave per destination row b: the row (re-sorted by (distance, id)) is
// merged with the offered sources in chunks of 64; sources already in the
// original row are dropped, repeated sources are kept as the reference does.
__global__ void __launch_bounds__(256) rin_merge_kernel(int32_t* __restrict__ ids, float* __restrict__ d, int64_t N,
                                                        int M, const uint32_t* __restrict__ off,
                                                        const unsigned long long* __restrict__ keys)
{
    __shared__ uint64_t L[4][2][kRinMaxM];
    __shared__ uint64_t C[4][64];
    __shared__ int32_t H[4][kRinHash];
    const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int64_t b = static_cast<int64_t>(blockIdx.x) * 4 + w;
    if (b >= N) return;
    const uint32_t lo = off[b], n = off[b + 1] - lo;
    if (n == 0) return;   // nothing offered: the row stays as it is

    for (int s = lane; s < kRinHash; s += 64) H[w][s] = -1;
    uint64_t e0 = kNoKey, e1 = kNoKey;
    if (lane < M) e0 = pack_key(d[b * M + lane], ids[b * M + lane]);
    if (lane + 64 < M) e1 = pack_key(d[b * M + lane + 64], ids[b * M + lane + 64]);
    wave_sync();
    constexpr uint32_t hmask = kRinHash - 1;
    auto hinsert = [&](int32_t x) {
        uint32_t h = (static_cast<uint32_t>(x) * 2654435761u) & hmask;
        while (true) {
            const int32_t old = atomicCAS(&H[w][h], -1, x);
            if (old == -1 || old == x) return;
            h = (h + 1) & hmask;
        }
    };
    auto hfind = [&](int32_t x) -> bool {
        uint32_t h = (static_cast<uint32_t>(x) * 2654435761u) & hmask;
        while (true) {
            const int32_t cur = H[w][h];
            if (cur == x) return true;
            if (cur == -1) return false;
            h = (h + 1) & hmask;
        }
    };
    if (lane < M && static_cast<int32_t>(e0) >= 0) hinsert(static_cast<int32_t>(e0));
    if (lane + 64 < M && static_cast<int32_t>(e1) >= 0) hinsert(static_cast<int32_t>(e1));
    wave_sort128_u64(e0, e1, lane);
    int cur = 0;
    if (lane < M) L[w][0][lane] = e0;
    if (lane + 64 < M) L[w][0][lane + 64] = e1;
    wave_sync();

    bool changed = false;   // uniform: only rows that take an offer are rewritten
    for (uint32_t c0 = 0; c0 < n; c0 += 64) {
        uint64_t key = kNoKey;
        const uint64_t thr = L[w][cur][M - 1];
        if (c0 + lane < n) {
            key = keys[lo + c0 + lane];
            if (key >= thr || hfind(static_cast<int32_t>(key))) key = kNoKey;
        }
        const uint64_t live = __ballot(key != kNoKey);
        if (live == 0) continue;
        changed = true;
        key = wave_sort64_u64(key, lane);
        const int nc = __popcll(live);
        C[w][lane] = key;
        wave_sync();
        // rank merge: row entries precede equal offered keys
        for (int k = lane; k < M; k += 64) {
            const uint64_t x = L[w][cur][k];
            int a = 0, z = nc;
            while (a < z) { const int m = (a + z) >> 1; if (C[w][m] < x) a = m + 1; else z = m; }
            if (k + a < M) L[w][cur ^ 1][k + a] = x;
        }
        if (lane < nc) {
            int a = 0, z = M;
            while (a < z) { const int m = (a + z) >> 1; if (L[w][cur][m] <= key) a = m + 1; else z = m; }
            if (lane + a < M) L[w][cur ^ 1][lane + a] = key;
        }
        wave_sync();
        cur ^= 1;
    }
    if (!changed) return;
    for (int k = lane; k < M; k += 64) {
        const uint64_t x = L[w][cur][k];
        ids[b * M + k] = static_cast<int32_t>(static_cast<uint32_t>(x));
        d[b * M + k] = o2f(static_cast<uint32_t>(x >> 32));
    }
}

static unsigned blocks_for(int64_t n, int per_block)
{
    return static_cast<unsigned>(ceil_div(n, per_block));
}

void launch_occlusion_prune(const float* X, int64_t N, int Dp, const int32_t* nb, int M, int max_deg, int32_t* out,
                            hipStream_t s)
{
    GT_REQUIRE(M >= 1 && M <= kOccMaxM, "occlusion prune: list length must be in [1, 128]");
    GT_REQUIRE(Dp % 32 == 0, "occlusion prune: padded dimension must be a multiple of 32");
    if (N <= 0) return;
    const dim3 grid(blocks_for(N, 4)), block(256);
    switch ((M + 31) / 32) {
    case 1: hipLaunchKernelGGL((occlusion_prune_kernel<1, 1>), grid, block, 0, s, X, N, Dp, nb, M, max_deg, out); break;
    case 2: hipLaunchKernelGGL((occlusion_prune_kernel<2, 2>), grid, block, 0, s, X, N, Dp, nb, M, max_deg, out); break;
    case 3: hipLaunchKernelGGL((occlusion_prune_kernel<3, 2>), grid, block, 0, s, X, N, Dp, nb, M, max_deg, out); break;
    default: hipLaunchKernelGGL((occlusion_prune_kernel<4, 2>), grid, block, 0, s, X, N, Dp, nb, M, max_deg, out); break;
    }
    GT_HIP(hipGetLastError());
}

void launch_rin_worst(const float* d, int64_t N, int M, float* worst, hipStream_t s)
{
    if (N <= 0) return;
    hipLaunchKernelGGL(rin_worst_kernel, dim3(blocks_for(N, 256)), dim3(256), 0, s, d, N, M, worst);
    GT_HIP(hipGetLastError());
}

void launch_rin_count(const int32_t* ids, const float* d, int64_t N, int M, const float* worst, uint32_t* cnt,
                      uint32_t* slot, int* err, hipStream_t s)
{
    const int64_t E = N * M;
    if (E <= 0) return;
    hipLaunchKernelGGL(rin_count_kernel, dim3(blocks_for(E, 256)), dim3(256), 0, s, ids, d, E, N, worst, cnt, slot,
                       err);
    GT_HIP(hipGetLastError());
}

void launch_rin_scatter(const int32_t* ids, const float* d, int64_t N, int M, const uint32_t* off,
                        const uint32_t* slot, unsigned long long* keys, hipStream_t s)
{
    const int64_t E = N * M;
    if (E <= 0) return;
    hipLaunchKernelGGL(rin_scatter_kernel, dim3(blocks_for(E, 256)), dim3(256), 0, s, ids, d, E, M, off, slot, keys);
    GT_HIP(hipGetLastError());
}

void launch_rin_merge(int32_t* ids, float* d, int64_t N, int M, const uint32_t* off, const unsigned long long* keys,
                      hipStream_t s)
{
    GT_REQUIRE(M >= 1 && M <= kRinMaxM, "reverse-edge insertion: list length must be in [1, 128]");
    if (N <= 0) return;
    hipLaunchKernelGGL(rin_merge_kernel, dim3(blocks_for(N, 4)), dim3(256), 0, s, ids, d, N, M, off, keys);
    GT_HIP(hipGetLastError());
}

}  // namespace gtann
