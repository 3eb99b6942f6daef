// knn_device.hpp -- device definitions shared by the kNN kernels
// (knn_kernels.hip: lists merged in the scan; knn_collect.hip: candidates
// collected under a threshold, then selected).
#pragma once

#include "gtann_common.hpp"

#include <cfloat>
#include <climits>
#include <cmath>
#include <type_traits>

namespace gtann {

typedef float floatx16 __attribute__((ext_vector_type(16)));
typedef int intx4 __attribute__((ext_vector_type(4)));
typedef int intx16 __attribute__((ext_vector_type(16)));

// f(std::integral_constant<int, I>{}) for I = 0 .. N-1: loop counters that
// are constants before any optimisation runs (register arrays indexed by
// them never become memory)
template <int I, int N, typename F>
__device__ __forceinline__ void static_for(F&& f)
{
    if constexpr (I < N) {
        f(std::integral_constant<int, I>{});
        static_for<I + 1, N>(f);
    }
}

// Waits until every vector memory access of this wave has completed: rows a
// wave stores (list rows, candidate slots) are loaded again by the same wave
// only after one of these waits.
__device__ __forceinline__ void wait_vmem() { __builtin_amdgcn_s_waitcnt(0x0F70); }   // vmcnt(0)

// Accumulator start of a row past the slice end: no dot product (|dot| <
// 2^22) lifts it to a query's pass floor.
constexpr int32_t kHalfPast = -(1 << 30);

// Integer pre-filter of the int8 kernels.  Every distance of those kernels
// is an exact integer below 2^24 (int8 rows, int32 sums, |p|^2 and |q|^2
// exact in fp32), and their MFMA accumulators start at -floor(|p|^2 / 2), so
// they end at v = dot - floor(|p|^2 / 2).  With T = thr - |q|^2, a row passes
// (L2) iff |p|^2 - 2 dot <= T, i.e. 2v - (|p|^2 mod 2) >= -T, which implies
// v >= -floor(T / 2): a tile none of whose v reach that floor holds no row
// that passes.  For the inner product d = -dot = -v, and a row passes iff
// v >= -thr.  No cap yet (FLT_MAX): every v passes; an invalid query (-inf):
// none does.
template <int METRIC>
__device__ __forceinline__ int32_t i8_pass_floor(float thr, float qn)
{
    if (thr > 6.0e7f) return INT_MIN;
    if (thr < -6.0e7f) return INT_MAX;
    return METRIC == 0 ? -static_cast<int32_t>(floorf((thr - qn) * 0.5f)) : -static_cast<int32_t>(floorf(thr));
}

// Inclusive prefix sum across the 64 lanes: row shifts by 1, 2, 4 and 8 sum
// within each row of 16 lanes, then rows 1 and 3 add the last lane of the row
// before them, rows 2 and 3 the last lane of row 1.
__device__ __forceinline__ int wave_incl_scan(int x)
{
    x += __builtin_amdgcn_update_dpp(0, x, 0x111, 0xf, 0xf, false);   // row_shr:1
    x += __builtin_amdgcn_update_dpp(0, x, 0x112, 0xf, 0xf, false);   // row_shr:2
    x += __builtin_amdgcn_update_dpp(0, x, 0x114, 0xf, 0xf, false);   // row_shr:4
    x += __builtin_amdgcn_update_dpp(0, x, 0x118, 0xf, 0xf, false);   // row_shr:8
    x += __builtin_amdgcn_update_dpp(0, x, 0x142, 0xa, 0xf, false);   // row_bcast:15
    x += __builtin_amdgcn_update_dpp(0, x, 0x143, 0xc, 0xf, false);   // row_bcast:31
    return x;
}

// ------------------------------------------------------------ sorting networks
//
// Keys are packed (distance, id) words (pack_key): distinct within a query,
// so every network below has one result.  A query's keys are held by two
// lanes, l and l ^ 32, which run the same networks on their own registers;
// the layers that pair a lane with its partner exchange registers through
// partner64.

// the value of x held by lane l ^ 32 (ds_bpermute: the exchange runs on the
// LDS unit; v_permlane32_swap + a select made the VALU-bound merges slower)
__device__ __forceinline__ uint32_t partner32(uint32_t x)
{
    return static_cast<uint32_t>(__shfl_xor(static_cast<int>(x), 32));
}
__device__ __forceinline__ uint64_t partner64(uint64_t x)
{
    return (static_cast<uint64_t>(partner32(static_cast<uint32_t>(x >> 32))) << 32) |
           partner32(static_cast<uint32_t>(x));
}

__device__ __forceinline__ void ce_up(uint64_t& a, uint64_t& b)
{
    const bool sw = b < a;
    const uint64_t lo = sw ? b : a;
    b = sw ? a : b;
    a = lo;
}

__device__ __forceinline__ void ce_up(float& a, float& b)
{
    const float lo = fminf(a, b);
    b = fmaxf(a, b);
    a = lo;
}

__device__ __forceinline__ uint64_t key_min(uint64_t a, uint64_t b) { return b < a ? b : a; }

// Batcher's odd-even merge sort network of N inputs (N a power of two),
// built at compile time so that every compare-exchange names fixed registers
struct CePair {
    int a, b;
};
template <int N>
struct BatcherNet {
    CePair p[N * N];
    int n;
    constexpr BatcherNet() : p{}, n(0)
    {
        for (int q = 1; q < N; q <<= 1)
            for (int k = q; k >= 1; k >>= 1)
                for (int j = k % q; j + k < N; j += 2 * k)
                    for (int i = 0; i < k && i + j + k < N; ++i)
                        if ((i + j) / (2 * q) == (i + j + k) / (2 * q)) {
                            p[n].a = i + j;
                            p[n].b = i + j + k;
                            ++n;
                        }
    }
};

template <typename K, int N>
__device__ __forceinline__ void oddeven_sort(K (&x)[N])
{
    constexpr BatcherNet<N> net{};
#pragma unroll
    for (int c = 0; c < net.n; ++c) ce_up(x[net.p[c].a], x[net.p[c].b]);
}

// a bitonic sequence of N keys into ascending order: layers of distance J,
// J / 2, ..., 1
template <typename K, int N, int J = N / 2>
__device__ __forceinline__ void bitonic_merge(K (&x)[N])
{
    if constexpr (J > 0) {
#pragma unroll
        for (int i = 0; i < N; ++i)
            if ((i & J) == 0) ce_up(x[i], x[i + J]);
        bitonic_merge<K, N, J / 2>(x);
    }
}

// A sorted list of 2 LM keys in the registers of a lane pair: lane l (l < 32)
// holds positions [0, LM), lane l + 32 positions [LM, 2 LM).
template <int LM>
struct PairList {
    uint64_t k[LM];
};

// Sorts 32 keys, 16 per lane in any order (kNoKey for empty slots), across
// the lane pair: afterwards lane l holds ranks 0..15 ascending, lane l + 32
// ranks 16..31 (16 per lane, then an element-wise min / max against the
// partner's keys reversed and a bitonic merge within each lane).
__device__ __forceinline__ void pair_sort32(uint64_t (&b)[16], bool hi)
{
    oddeven_sort(b);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const uint64_t pa = partner64(b[15 - i]), pb = partner64(b[i]);
        const bool la = pa < b[i], lb = pb < b[15 - i];
        b[i] = (la != hi) ? pa : b[i];
        b[15 - i] = (lb != hi) ? pb : b[15 - i];
    }
    bitonic_merge(b);
}

// The first 32 keys of an empty list: the list becomes them, sorted.
template <int LM>
__device__ __forceinline__ void pair_first32(uint64_t (&b)[16], PairList<LM>& PL, bool hi)
{
    static_assert(LM == 16 || LM == 32, "lists of 32 or 64 keys per pair");
    pair_sort32(b, hi);
    if constexpr (LM == 32) {
        // positions 0..31 in lane l: its ranks 0..15, then the partner's 16..31
#pragma unroll
        for (int k = 0; k < 16; ++k) {
            const uint64_t t = partner64(b[k]);
            PL.k[k] = hi ? kNoKey : b[k];
            PL.k[16 + k] = hi ? kNoKey : t;
        }
    } else {
#pragma unroll
        for (int k = 0; k < 16; ++k) PL.k[k] = b[k];
    }
}

// Merges 32 keys, 16 per lane in any order (kNoKey for empty slots), into
// the pair's list, which keeps the 2 LM smallest keys of both, sorted.  The
// 32 keys are sorted (pair_sort32), laid against the list's tail in reverse
// (the element-wise minimum of an ascending and a descending sequence is
// bitonic and holds the 2 LM smallest keys of both), and the result is
// sorted by a bitonic merge whose first layer pairs each lane with its
// partner.  Both lanes of every pair must call it.
template <int LM>
__device__ __forceinline__ void pair_merge32(uint64_t (&b)[16], PairList<LM>& PL, bool hi)
{
    static_assert(LM == 16 || LM == 32, "lists of 32 or 64 keys per pair");
    uint64_t (&L)[LM] = PL.k;
    pair_sort32(b, hi);
    if constexpr (LM == 32) {
        // positions 32 + k take min(list, keys[31 - k]): the upper lane's
        // own keys reversed, then the lower lane's
#pragma unroll
        for (int k = 0; k < 16; ++k) L[k] = hi ? key_min(L[k], b[15 - k]) : L[k];
#pragma unroll
        for (int k = 16; k < 32; ++k) {
            const uint64_t t = partner64(b[31 - k]);
            L[k] = hi ? key_min(L[k], t) : L[k];
        }
    } else {
        // positions i take min(list, keys[31 - i]): the partner's keys reversed
#pragma unroll
        for (int k = 0; k < 16; ++k) L[k] = key_min(L[k], partner64(b[15 - k]));
    }
#pragma unroll
    for (int i = 0; i < LM; ++i) {
        const uint64_t o = partner64(L[i]);
        const bool lt = o < L[i];
        L[i] = (lt != hi) ? o : L[i];
    }
    bitonic_merge(L);
}

}  // namespace gtann
