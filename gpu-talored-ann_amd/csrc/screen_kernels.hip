// screen_kernels.hip -- bf16 screen ahead of a seeded fp32 collect pass.
//
// A seeded pass over fp32 rows collects, for every query q of a 128-query
// work item, the keys of the item's pool at or below q's running M-th
// distance T_q, then selects and merges them (knn_f32_collect_kernel).  The
// screen computes every (q, p) pair of the item on the bf16 matrix cores
// (v_mfma_f32_32x32x16_bf16: rows rounded to bf16, fp32 sums) and keeps the
// pool rows p whose bf16 key minus a rigorous bound e(q, p) is at most T_q
// for some query of the item.  e bounds the gap between the bf16 key and the
// fp32 path's key, so every row whose fp32 key is at or below T_q is kept;
// the union of kept rows, in pool order, becomes the item's pool for the fp32
// collect pass, which therefore collects exactly the keys the full pool would
// give it (its keys are per pair and ordered by (key, id), so neither the
// rows it no longer visits nor the visiting order change a list): the merged
// table is the unscreened pass's bit for bit.
//
// The bound.  S = sum_i |q_i p_i| <= |q| |p| (Cauchy-Schwarz).  Rounding a
// row to bf16 moves each element by at most 2^-8 of itself, so a product of
// two rounded elements is within (2^-7 + 2^-16) of the exact one; the bf16
// products are exact in fp32, and either path's fp32 sums over D <= 160 terms
// (in any order, each add within 2^-23 of its result: truncating adds
// included) add at most D 2^-23 (1 + 2^-7) S < 2^-15.6 S each.  The two dot
// products thus differ by less than (2^-7 + 2^-14) S < c S with
// c = 2^-7 + 2^-11, which leaves 2^-12 S for matrix-core sums coarser than
// that.  The fp32 key's own roundings
// (|q|^2 + |p|^2 then one fma, results of at most 2 (|q|^2 + |p|^2)) and the
// roundings of the screen's test below add less than 2^-19 (|q|^2 + |p|^2) for
// L2; 2^-60 absolute covers flushed denormal products.
//   L2 (key |q|^2 + |p|^2 - 2 q.p):  e = 2 c |q||p| + 2^-19 (|q|^2 + |p|^2)
//   IP (key -q.p):                    e = (c + 2^-19) |q||p|
// |x| is sqrt of the fp32 |x|^2 both paths use (within 2^-23 relative of the
// true norm, far inside the 2^-11 spare of c).  The test "bf16 key - e <= T"
// is evaluated as
//   L2: fma(2, d, fma(2 c |q|, |p|, -(1 - 2^-19) |p|^2)) >= (1 - 2^-19) |q|^2 - T - 2^-60
//   IP: fma((c + 2^-19) |q|, |p|, d)                      >= -T - 2^-60
// (d the bf16 dot): two and one vector instructions per pair before the
// compare, the pool row's two terms staged with its bf16 row.  T = +inf
// keeps every row.
#include "gtann_common.hpp"

#include <algorithm>

namespace gtann {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float floatx16 __attribute__((ext_vector_type(16)));

constexpr int kScreenMaxPool = 32768;   // pool rows an item's LDS bitmap covers
constexpr float kScreenC = 0x1p-7f + 0x1p-11f;
constexpr float kScreenR = 0x1p-19f;
constexpr float kScreenA = 0x1p-60f;

// fp32 rows (stride Dp) -> bf16 rows (stride Dp), rounded to nearest even
__global__ void __launch_bounds__(256) screen_bf16_kernel(const float4* __restrict__ X, int64_t n4,
                                                         uint2* __restrict__ Xb)
{
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; i < n4;
         i += static_cast<int64_t>(gridDim.x) * 256) {
        const float4 v = X[i];
        const float f[4] = {v.x, v.y, v.z, v.w};
        uint32_t o[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const uint32_t u = __float_as_uint(f[e]);
            o[e] = (u & 0x7FFFFFFFu) > 0x7F800000u ? ((u >> 16) | 0x40u)   // NaN stays NaN
                                                   : (u + 0x7FFFu + ((u >> 16) & 1u)) >> 16;
        }
        Xb[i] = make_uint2(o[0] | (o[1] << 16), o[2] | (o[3] << 16));
    }
}

// One block per work item (4 waves of 32 queries; lanes j and j + 32 hold
// query j's dims 16 s + 8 h + [0, 8) of step s, h = lane / 32).  Pool tiles
// of 32 rows are staged through LDS, double buffered (the next tile's loads
// in flight during a tile's MFMAs).  With the queries as the MFMA's rows, a
// tile's accumulator element 4 g + e of lane (j, h) is pool row j against
// query 8 g + 4 h + e; the 16 compares' lane masks OR into the tile's
// admitted rows (bit j from lanes j and j + 32), which each wave ORs into
// word t of the item's LDS bitmap; the set bits, in pool order, become the
// item's union at union_rows[ubase[item] ...).
template <int DP, int METRIC>
__global__ void __launch_bounds__(256) knn_screen_kernel(const WorkItem* __restrict__ items,
                                                         const int64_t* __restrict__ ubase,
                                                         const int32_t* __restrict__ q_rows,
                                                         const int32_t* __restrict__ p_rows,
                                                         const uint16_t* __restrict__ Xb, const float* __restrict__ nrm,
                                                         const float* __restrict__ seed_d, int seed_ld,
                                                         int32_t* __restrict__ union_rows,
                                                         WorkItem* __restrict__ items_out,
                                                         unsigned long long* __restrict__ pairs_done)
{
    constexpr int KS = DP / 16;          // MFMA steps per tile
    constexpr int RS = DP + 8;           // LDS row stride (bf16 elements): rows on distinct bank groups
    constexpr int U4_ROW = DP / 8;       // 16-byte pieces per row
    constexpr int U4_TILE = kPoolTile * U4_ROW;
    constexpr int U4_THREAD = (U4_TILE + 255) / 256;
    constexpr int WPT = kScreenMaxPool / 32 / 256;   // bitmap words per thread in the compaction
    static_assert(DP % 16 == 0 && kPoolTile == 32, "bf16 steps of 16 dims, one bitmap word per tile");
    __shared__ __align__(16) uint16_t tile[2][kPoolTile][RS];
    __shared__ float tpr[2][kPoolTile];   // |p|
    __shared__ float tpm[2][kPoolTile];   // -(1 - R) |p|^2
    __shared__ uint32_t bits[kScreenMaxPool / 32];
    __shared__ uint32_t wsum[kWaves];

    const int item_idx = blockIdx.x;
    const WorkItem it = items[item_idx];
    const int tid = threadIdx.x;
    if (it.q_count <= 0) {   // padding
        if (tid == 0) items_out[item_idx] = it;
        return;
    }
    const int w = tid >> 6, lane = tid & 63, j = lane & 31, h = lane >> 5;
    const int pc = it.p_count;
    const int ntiles = (pc + kPoolTile - 1) / kPoolTile;
    for (int i = tid; i < ntiles; i += 256) bits[i] = 0u;

    const int qlocal = w * kQueriesPerWave + j;
    const bool qvalid = qlocal < it.q_count;
    const int64_t qi = it.q_begin + qlocal;
    const int32_t qrow = qvalid ? (q_rows ? q_rows[qi] : static_cast<int32_t>(qi)) : 0;
    const int64_t orow_seed = it.out_base >= 0 ? it.out_base + qlocal : static_cast<int64_t>(qrow);
    const float T = qvalid ? seed_d[orow_seed * seed_ld + seed_ld - 1] : 0.f;
    const float qn = nrm[qrow];
    const float qr = sqrtf(qn);
    const float cq = METRIC == 0 ? 2.f * kScreenC * qr : (kScreenC + kScreenR) * qr;
    // an invalid query admits nothing (y >= +inf fails for every finite y)
    const float qa = !qvalid ? INFINITY : METRIC == 0 ? qn * (1.f - kScreenR) - T - kScreenA : -T - kScreenA;
    // the constants of the queries this lane's accumulator elements hold
    // (element 4 g + e: query 8 g + 4 h + e of the wave)
    float qa_r[16], cq_r[16];
#pragma unroll
    for (int r = 0; r < 16; ++r) {
        const int src = 8 * (r >> 2) + 4 * h + (r & 3);
        qa_r[r] = __shfl(qa, src);
        cq_r[r] = __shfl(cq, src);
    }
    bf16x8 qf[KS];
    {
        const uint4* src = reinterpret_cast<const uint4*>(Xb + static_cast<int64_t>(qrow) * DP + 8 * h);
#pragma unroll
        for (int s = 0; s < KS; ++s) qf[s] = __builtin_bit_cast(bf16x8, src[2 * s]);
    }

    uint4 pre[U4_THREAD];
    auto load_tile = [&](int t) __attribute__((always_inline)) {
#pragma unroll
        for (int u = 0; u < U4_THREAD; ++u) {
            const int e = tid + 256 * u;
            pre[u] = make_uint4(0u, 0u, 0u, 0u);
            if (e < U4_TILE) {
                const int p = t * kPoolTile + e / U4_ROW;
                if (p < pc) {
                    const int32_t row = p_rows[it.p_begin + p];
                    pre[u] = reinterpret_cast<const uint4*>(Xb + static_cast<int64_t>(row) * DP)[e % U4_ROW];
                }
            }
        }
    };
    auto store_tile = [&](int t, int buf) __attribute__((always_inline)) {
#pragma unroll
        for (int u = 0; u < U4_THREAD; ++u) {
            const int e = tid + 256 * u;
            if (e < U4_TILE) *reinterpret_cast<uint4*>(&tile[buf][e / U4_ROW][8 * (e % U4_ROW)]) = pre[u];
        }
        if (tid < kPoolTile) {
            const int p = t * kPoolTile + tid;
            const float pn = p < pc ? nrm[p_rows[it.p_begin + p]] : 0.f;
            tpr[buf][tid] = sqrtf(pn);
            tpm[buf][tid] = -(1.f - kScreenR) * pn;
        }
    };
    if (ntiles > 0) {
        load_tile(0);
        store_tile(0, 0);
    }
    __syncthreads();
    for (int t = 0; t < ntiles; ++t) {
        const int buf = t & 1;
        if (t + 1 < ntiles) load_tile(t + 1);
        floatx16 acc;
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[r] = 0.f;
        // queries as A (rows), pool rows as B (columns): lane (j, h) ends
        // with pool row j against queries 8 g + 4 h + e
        const uint16_t* brow = &tile[buf][j][8 * h];
#pragma unroll
        for (int s = 0; s < KS; ++s) {
            const bf16x8 bv = __builtin_bit_cast(bf16x8, *reinterpret_cast<const uint4*>(brow + 16 * s));
            acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(qf[s], bv, acc, 0, 0, 0);
        }
        const float pr = tpr[buf][j], pm = tpm[buf][j];
        uint64_t m = 0u;   // lanes whose pool row some query admits
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const float y = METRIC == 0 ? fmaf(2.f, acc[r], fmaf(cq_r[r], pr, pm)) : fmaf(cq_r[r], pr, acc[r]);
            m |= __ballot(y >= qa_r[r]);
        }
        uint32_t tm = static_cast<uint32_t>(m) | static_cast<uint32_t>(m >> 32);   // bit j: pool row j
        const int left = pc - t * kPoolTile;
        if (left < kPoolTile) tm &= (1u << left) - 1u;
        if (lane == 0 && tm) atomicOr(&bits[t], tm);
        if (t + 1 < ntiles) store_tile(t + 1, buf ^ 1);
        __syncthreads();
    }
    // the set bits, in order, as row ids
    uint32_t cnt = 0u;
#pragma unroll
    for (int u = 0; u < WPT; ++u) {
        const int wi = tid * WPT + u;
        cnt += wi < ntiles ? static_cast<uint32_t>(__popc(bits[wi])) : 0u;
    }
    uint32_t inc = cnt;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const uint32_t x = __shfl_up(inc, o);
        if (lane >= o) inc += x;
    }
    if (lane == 63) wsum[w] = inc;
    __syncthreads();
    uint32_t off = inc - cnt;
    for (int q = 0; q < w; ++q) off += wsum[q];
    const int64_t base = ubase[item_idx];
#pragma unroll
    for (int u = 0; u < WPT; ++u) {
        const int wi = tid * WPT + u;
        uint32_t b = wi < ntiles ? bits[wi] : 0u;
        while (b) {
            const int k = __ffs(b) - 1;
            b &= b - 1u;
            union_rows[base + off++] = p_rows[it.p_begin + wi * 32 + k];
        }
    }
    if (tid == 0) {
        WorkItem o = it;
        o.p_begin = base;
        o.p_count = static_cast<int32_t>(wsum[0] + wsum[1] + wsum[2] + wsum[3]);
        o.p_rot = 0;
        items_out[item_idx] = o;
        if (pairs_done)
            atomicAdd(pairs_done, static_cast<unsigned long long>(o.p_count) * static_cast<unsigned>(o.q_count));
    }
}

bool screen_supported(int Dp, int64_t max_pool)
{
    return (Dp == 32 || Dp == 64 || Dp == 96 || Dp == 128 || Dp == 160) && max_pool <= kScreenMaxPool;
}

void launch_screen_bf16(const float* X, int64_t N, int Dp, uint16_t* Xb, hipStream_t s)
{
    GT_REQUIRE(Dp % 4 == 0, "screen: rows of whole float4s");
    const int64_t n4 = N * Dp / 4;
    if (n4 <= 0) return;
    const unsigned grid = static_cast<unsigned>(std::min<int64_t>(ceil_div(n4, int64_t(256)), 8192));
    hipLaunchKernelGGL(screen_bf16_kernel, dim3(grid), dim3(256), 0, s, reinterpret_cast<const float4*>(X), n4,
                       reinterpret_cast<uint2*>(Xb));
    GT_HIP(hipGetLastError());
}

// items: n_items work items of a seeded pass (every pool at most
// kScreenMaxPool rows); ubase[i]: item i's first slot of union_rows, which
// holds at least its pool count from there; items_out: the items with their
// unions as pools.  Xb: bf16 rows (stride Dp) of the matrix the q_rows and
// p_rows index, nrm its fp32 |x|^2.  pairs_done (optional) += the (query,
// union row) pairs left to the fp32 pass.
void launch_screen(const WorkItem* items, int n_items, const int64_t* ubase, const int32_t* q_rows,
                   const int32_t* p_rows, const uint16_t* Xb, const float* nrm, int Dp, int metric,
                   const float* seed_d, int seed_ld, int32_t* union_rows, WorkItem* items_out,
                   unsigned long long* pairs_done, hipStream_t s)
{
    GT_REQUIRE(screen_supported(Dp, 0), "screen: padded dimension not supported");
    GT_REQUIRE(seed_d != nullptr && seed_ld > 0, "screen: a seeded pass only");
    if (n_items <= 0) return;
#define GT_SCR(DPV)                                                                                           \
    do {                                                                                                      \
        if (metric == 0)                                                                                      \
            hipLaunchKernelGGL((knn_screen_kernel<DPV, 0>), dim3(n_items), dim3(256), 0, s, items, ubase,     \
                               q_rows, p_rows, Xb, nrm, seed_d, seed_ld, union_rows, items_out, pairs_done);            \
        else                                                                                                  \
            hipLaunchKernelGGL((knn_screen_kernel<DPV, 1>), dim3(n_items), dim3(256), 0, s, items, ubase,     \
                               q_rows, p_rows, Xb, nrm, seed_d, seed_ld, union_rows, items_out, pairs_done);            \
    } while (0)
    switch (Dp) {
    case 32: GT_SCR(32); break;
    case 64: GT_SCR(64); break;
    case 96: GT_SCR(96); break;
    case 128: GT_SCR(128); break;
    default: GT_SCR(160); break;
    }
#undef GT_SCR
    GT_HIP(hipGetLastError());
}

}  // namespace gtann
