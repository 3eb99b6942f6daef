// search_kernel.hip -- beam (ef) search over a graph on gfx950.
//
// One wave per query runs the reference's sequential best-first search
// (bd/search.py:20-90, graph_search_single) step for step, with the work of
// each step spread over the 64 lanes:
//   * pop: the candidate with the smallest (distance, id) -- every lane scans
//     its strided share of the LDS candidate array, a wave min picks the key;
//   * expand: lane j takes neighbour j of the popped row (rows longer than 64
//     in chunks), drops ids outside [0, N) and repeats of an earlier lane in
//     the same row, tests-and-sets the visited table, and computes the
//     distance of its new point (one row per lane, four fmaf chains by
//     dimension mod 4, the CPU restatement's order, so the value is bit for
//     bit the same);
//   * best list: new points are applied in row order -- appended while the
//     list is short, then each strictly closer point replaces the first slot
//     holding the maximum (np.argmax), the maximum recomputed by a wave max
//     after every replacement.
// The visited set is an LDS hash table (open addressing, linear probing);
// a query that would fill it past 3/4 stops with status 1 and the host runs
// it again with a per-wave bitmap of N bits in HBM.  Candidates that can no
// longer be popped (distance beyond a full best list's maximum) are not
// stored, and are dropped when the array fills; status 2 reports a query
// whose live candidates still do not fit (more than the capacity tie at the
// maximum), which the host turns into an error.
#include "gtann_common.hpp"

#include <cfloat>

namespace gtann {


__device__ __forceinline__ int lanes_below(uint64_t m)
{
    return __builtin_amdgcn_mbcnt_hi(static_cast<uint32_t>(m >> 32),
                                     __builtin_amdgcn_mbcnt_lo(static_cast<uint32_t>(m), 0u));
}

__device__ __forceinline__ float readlane_f(float v, int l)
{
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), l));
}

__global__ void __launch_bounds__(64) graph_search_kernel(SearchArgs a)
{
    extern __shared__ __align__(16) unsigned char smem[];
    uint64_t* ck = reinterpret_cast<uint64_t*>(smem);                 // candidate keys (d, id)
    float* bd = reinterpret_cast<float*>(ck + a.CC);                  // best list: distance per slot
    int32_t* bi = reinterpret_cast<int32_t*>(bd + a.efr);             // best list: id per slot
    float* qv = reinterpret_cast<float*>(bi + a.efr);                 // query row
    int32_t* hs = reinterpret_cast<int32_t*>(qv + a.Dp);              // visited table

    const int lane = threadIdx.x;
    const uint32_t N = static_cast<uint32_t>(a.N);
    uint32_t* bm = a.bitmap ? a.bitmap + static_cast<int64_t>(blockIdx.x) * a.bm_words : nullptr;
    const int hshift = a.H ? 32 - (31 - __clz(a.H)) : 0;
    const int hlimit = a.H - a.H / 4;

    for (int64_t r = blockIdx.x; r < a.n_run; r += gridDim.x) {
        const int64_t q = a.q_list ? a.q_list[r] : r;
        for (int k = lane; k < a.Dp / 4; k += 64)
            reinterpret_cast<float4*>(qv)[k] = reinterpret_cast<const float4*>(a.Q + q * a.Dp)[k];
        for (int k = lane; k < a.H; k += 64) hs[k] = -1;
        wave_sync();

        int nb = 0;          // best list length
        int nc = 0;          // candidates
        int nvis = 0;        // visited points
        int st = 0;
        int nexp = 0;
        float worst = 0.f;   // maximum of the best list once it holds ef points
        int wpos = 0;        // its first slot

        auto recompute_worst = [&]() {
            uint64_t best = 0;
            for (int i = lane; i < a.ef; i += 64) {
                const uint64_t k = (static_cast<uint64_t>(f2o(bd[i])) << 32) | static_cast<uint32_t>(~i);
                best = k > best ? k : best;
            }
#pragma unroll
            for (int o = 32; o > 0; o >>= 1) {
                const uint64_t t = shfl_xor_u64(best, o);
                best = t > best ? t : best;
            }
            worst = o2f(static_cast<uint32_t>(best >> 32));
            wpos = static_cast<int>(~static_cast<uint32_t>(best));
        };

        // Four partial sums, one per dimension mod 4 (the float4 lanes), over
        // the zero-padded row (padding adds exact zeros), combined as
        // (s0 + s1) + (s2 + s3).  Up to 32 float4 loads are issued before the
        // first use, so a row of up to 128 dimensions costs one memory latency.
        auto distance = [&](uint32_t v) -> float {
            const float4* xr = reinterpret_cast<const float4*>(a.X + static_cast<int64_t>(v) * a.Dp);
            const float4* qr = reinterpret_cast<const float4*>(qv);
            const int n4 = a.Dp >> 2;
            float s0 = 0.f, s1 = 0.f, s2 = 0.f, s3 = 0.f;
            for (int base = 0; base < n4; base += 32) {
                float4 x[32];
#pragma unroll
                for (int k = 0; k < 32; ++k) x[k] = xr[min(base + k, n4 - 1)];
#pragma unroll
                for (int k = 0; k < 32; ++k) {
                    const bool in = base + k < n4;
                    const float4 y = qr[min(base + k, n4 - 1)];
                    if (a.metric == 0) {
                        const float t0 = in ? y.x - x[k].x : 0.f, t1 = in ? y.y - x[k].y : 0.f;
                        const float t2 = in ? y.z - x[k].z : 0.f, t3 = in ? y.w - x[k].w : 0.f;
                        s0 = fmaf(t0, t0, s0);
                        s1 = fmaf(t1, t1, s1);
                        s2 = fmaf(t2, t2, s2);
                        s3 = fmaf(t3, t3, s3);
                    } else {
                        s0 = fmaf(in ? y.x : 0.f, x[k].x, s0);
                        s1 = fmaf(in ? y.y : 0.f, x[k].y, s1);
                        s2 = fmaf(in ? y.z : 0.f, x[k].z, s2);
                        s3 = fmaf(in ? y.w : 0.f, x[k].w, s3);
                    }
                }
            }
            const float s = (s0 + s1) + (s2 + s3);
            return a.metric == 0 ? s : -s;
        };

        // Visits the ids held by the lanes in lane order (the reference's
        // loop order); lanes without an id hold 0xFFFFFFFF.  false = the
        // query stopped (st set).
        auto visit = [&](uint32_t v) -> bool {
            bool fresh = v < N;
            const uint64_t valid = __ballot(fresh);
            for (uint64_t m = valid; m; m &= m - 1) {     // repeats of an earlier lane
                const int i = __ffsll(static_cast<unsigned long long>(m)) - 1;
                const uint32_t o = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(v), i));
                fresh = fresh && !(lane > i && o == v);
            }
            bool isnew = false;
            if (fresh) {
                if (bm) {
                    const uint32_t bit = 1u << (v & 31u);
                    isnew = (atomicOr(&bm[v >> 5], bit) & bit) == 0u;
                } else {
                    uint32_t h = (v * 2654435761u) >> hshift;
                    for (;;) {
                        const int32_t old = atomicCAS(&hs[h], -1, static_cast<int32_t>(v));
                        if (old == -1) { isnew = true; break; }
                        if (old == static_cast<int32_t>(v)) break;
                        h = (h + 1u) & static_cast<uint32_t>(a.H - 1);
                    }
                }
            }
            const uint64_t newm = __ballot(isnew);
            if (!newm) return true;
            nvis += __popcll(newm);
            if (!bm && nvis > hlimit) { st = 1; return false; }

            const float dv = isnew ? distance(v) : 0.f;

            // candidates: a point beyond a full list's maximum is never popped
            const bool full0 = nb >= a.ef;
            const float worst0 = worst;
            const bool push = isnew && !(full0 && dv > worst0);
            const uint64_t pm = __ballot(push);
            const int cnt = __popcll(pm);
            if (nc + cnt > a.CC) {
                if (full0) {
                    int out = 0;
                    for (int base = 0; base < nc; base += 64) {
                        const int i = base + lane;
                        const uint64_t k = i < nc ? ck[i] : kNoKey;
                        const bool keep = i < nc && o2f(static_cast<uint32_t>(k >> 32)) <= worst0;
                        const uint64_t km = __ballot(keep);
                        wave_sync();
                        if (keep) ck[out + lanes_below(km)] = k;
                        out += __popcll(km);
                        wave_sync();
                    }
                    nc = out;
                }
                if (nc + cnt > a.CC) { st = 2; return false; }
            }
            if (push) ck[nc + lanes_below(pm)] = pack_key(dv, static_cast<int32_t>(v));
            nc += cnt;

            // best list, in lane order
            const int room = a.ef - nb;
            const int rank = lanes_below(newm);
            if (isnew && rank < room) {
                bd[nb + rank] = dv;
                bi[nb + rank] = static_cast<int32_t>(v);
            }
            const int app = min(__popcll(newm), room);
            nb += app;
            wave_sync();
            if (app > 0 && nb == a.ef) recompute_worst();
            uint64_t rest = __ballot(isnew && rank >= room);
            while (rest) {
                const uint64_t m = rest & __ballot(dv < worst);
                if (!m) break;
                const int l = __ffsll(static_cast<unsigned long long>(m)) - 1;
                const float dl = readlane_f(dv, l);
                const int32_t vl = __builtin_amdgcn_readlane(static_cast<int>(v), l);
                if (lane == 0) {
                    bd[wpos] = dl;
                    bi[wpos] = vl;
                }
                wave_sync();
                recompute_worst();
                rest &= ~((2ull << l) - 1ull);
            }
            wave_sync();
            return true;
        };

        // entry points, then best-first expansion
        bool ok = visit(lane < a.n_entry ? static_cast<uint32_t>(a.entries[q * a.n_entry + lane]) : 0xFFFFFFFFu);
        while (ok) {
            uint64_t mk = kNoKey;
            int ms = 0;
            for (int i = lane; i < nc; i += 64) {
                const uint64_t k = ck[i];
                if (k < mk) { mk = k; ms = i; }
            }
            uint64_t m = mk;
#pragma unroll
            for (int o = 32; o > 0; o >>= 1) {
                const uint64_t t = shfl_xor_u64(m, o);
                m = t < m ? t : m;
            }
            if (m == kNoKey) break;
            const int owner = __ffsll(static_cast<unsigned long long>(__ballot(mk == m))) - 1;
            const int slot = __builtin_amdgcn_readlane(ms, owner);
            wave_sync();
            if (lane == 0) ck[slot] = ck[nc - 1];
            --nc;
            wave_sync();
            const uint32_t u = static_cast<uint32_t>(m);
            if (nb >= a.ef && o2f(static_cast<uint32_t>(m >> 32)) > worst) break;
            ++nexp;
            for (int c = 0; c < a.deg && ok; c += 64) {
                const int j = c + lane;
                ok = visit(j < a.deg ? a.graph[static_cast<int64_t>(u) * a.deg + j] : 0xFFFFFFFFu);
            }
        }

        if (st == 0) {
            // the best list in (distance, slot) order: rank by counting
            for (int i = lane; i < nb; i += 64) {
                const float di = bd[i];
                int rk = 0;
                for (int j = 0; j < nb; ++j) {
                    const float dj = bd[j];
                    rk += (dj < di || (dj == di && j < i)) ? 1 : 0;
                }
                if (rk < a.topk) {
                    a.out_ids[q * a.topk + rk] = bi[i];
                    a.out_d[q * a.topk + rk] = a.metric == 1 ? -di : di;
                }
            }
            for (int t = nb + lane; t < a.topk; t += 64) {
                a.out_ids[q * a.topk + t] = -1;
                a.out_d[q * a.topk + t] = a.metric == 1 ? -INFINITY : INFINITY;
            }
        }
        if (lane == 0) {
            a.status[q] = st;
            a.expansions[q] = nexp;
            a.visits[q] = nvis;
        }
        if (bm) {
            for (int64_t k = lane; k < a.bm_words; k += 64) bm[k] = 0u;
            __threadfence();
        }
        wave_sync();
    }
}

size_t search_lds_bytes(int CC, int efr, int Dp, int H)
{
    return static_cast<size_t>(CC) * 8 + static_cast<size_t>(efr) * 8 + static_cast<size_t>(Dp) * 4 +
           static_cast<size_t>(H) * 4;
}

void launch_graph_search(const SearchArgs& a, int64_t grid, hipStream_t s)
{
    if (a.n_run <= 0) return;
    const size_t lds = search_lds_bytes(a.CC, a.efr, a.Dp, a.H);
    GT_REQUIRE(lds <= 65536, "search: per-query LDS exceeds 64 KiB (ef or D too large)");
    GT_REQUIRE(a.H == 0 || (a.H >= 512 && (a.H & (a.H - 1)) == 0), "search: visited table size");
    GT_REQUIRE(a.n_entry >= 1 && a.n_entry <= 64, "search: 1 <= entry points <= 64");
    GT_REQUIRE(grid >= 1 && grid <= (int64_t(1) << 31) - 1, "search: grid");
    hipLaunchKernelGGL(graph_search_kernel, dim3(static_cast<unsigned>(grid)), dim3(64), lds, s, a);
    GT_HIP(hipGetLastError());
}

}  // namespace gtann
