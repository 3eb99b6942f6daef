// graph_kernels.hip -- integer graph stages of the build on gfx950:
// sanitize, CAGRA rank-based detour-count prune, reverse-edge merge,
// cross-round list merge, id translation, plus layout helpers.
//
// All of them are deterministic: no result depends on the order in which
// atomics land (atomics only count, or fill slots that are re-ordered by a
// total key before use).
#include "gtann_common.hpp"

#include <climits>
#include <cmath>

namespace gtann {

// ------------------------------------------------------------------ layout

template <typename T>
__global__ void pad_convert_kernel(const T* __restrict__ src, float* __restrict__ dst, int64_t N, int D, int Dp)
{
    const int64_t total = N * Dp;
    for (int64_t e = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; e < total;
         e += static_cast<int64_t>(gridDim.x) * blockDim.x) {
        const int64_t r = e / Dp;
        const int c = static_cast<int>(e - r * Dp);
        dst[e] = c < D ? static_cast<float>(src[r * D + c]) : 0.f;
    }
}

// int8 rows for the int8 MFMA kernel: uint8 inputs are shifted by -128 (L2
// distances do not change under a common shift), int8 inputs copied; zero
// padded to Dp bytes.
template <typename T>
__global__ void pad_i8_kernel(const T* __restrict__ src, int8_t* __restrict__ dst, int64_t N, int D, int Dp, int shift)
{
    const int64_t total = N * Dp;
    for (int64_t e = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; e < total;
         e += static_cast<int64_t>(gridDim.x) * blockDim.x) {
        const int64_t r = e / Dp;
        const int c = static_cast<int>(e - r * Dp);
        dst[e] = c < D ? static_cast<int8_t>(static_cast<int>(src[r * D + c]) - shift) : int8_t(0);
    }
}

// One pass over integer-typed rows (D <= Dp <= 256): the float copy and the
// int8 copy (minus shift: 128 for uint8, 0 for int8), both zero padded to
// Dp, and both squared norms.  The norms are integers below 2^24, so they
// are exact in float whatever the summation order.  2^lpr_log2 lanes per row
// (at least Dp / 4), four columns per lane.
template <typename T, bool VEC>
__global__ void __launch_bounds__(256) prepare_int_kernel(const T* __restrict__ src, int64_t N, int D, int Dp,
                                                          int shift, int lpr_log2, float* __restrict__ xf,
                                                          float* __restrict__ nf, int8_t* __restrict__ x8,
                                                          float* __restrict__ n8)
{
    const int64_t gt = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
    const int64_t row = gt >> lpr_log2;
    const int c0 = 4 * static_cast<int>(gt & ((1 << lpr_log2) - 1));
    int sf = 0, s8 = 0;
    if (row < N && c0 < Dp) {
        int v[4];
        if constexpr (VEC) {
            // D % 4 == 0: the four columns are one aligned word, all in the row or all padding
            uint32_t wv = 0;
            if (c0 < D) wv = *reinterpret_cast<const uint32_t*>(src + row * D + c0);
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const uint32_t b = (wv >> (8 * u)) & 0xffu;
                v[u] = sizeof(T) == 1 && static_cast<T>(-1) < 0 ? static_cast<int>(static_cast<int8_t>(b))
                                                                 : static_cast<int>(b);
            }
        } else {
#pragma unroll
            for (int u = 0; u < 4; ++u) v[u] = c0 + u < D ? static_cast<int>(src[row * D + c0 + u]) : 0;
        }
        uint32_t q = 0;
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const int qv = c0 + u < D ? v[u] - shift : 0;
            sf += v[u] * v[u];
            s8 += qv * qv;
            q |= (static_cast<uint32_t>(qv) & 0xffu) << (8 * u);
        }
        *reinterpret_cast<float4*>(xf + row * Dp + c0) =
            make_float4(static_cast<float>(v[0]), static_cast<float>(v[1]), static_cast<float>(v[2]),
                        static_cast<float>(v[3]));
        *reinterpret_cast<uint32_t*>(x8 + row * Dp + c0) = q;
    }
    for (int o = 1 << (lpr_log2 - 1); o > 0; o >>= 1) {
        sf += __shfl_xor(sf, o);
        s8 += __shfl_xor(s8, o);
    }
    if (row < N && c0 == 0) {
        nf[row] = static_cast<float>(sf);
        n8[row] = static_cast<float>(s8);
    }
}

// int8 copy of float rows (centroids of an integer dataset): the value
// minus the dataset's shift, rounded and clamped; padding stays 0.
__global__ void quantize_i8_kernel(const float* __restrict__ src, int64_t N, int D, int Dp, int shift,
                                   int8_t* __restrict__ dst)
{
    const int64_t e = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (e >= N * Dp) return;
    const int c = static_cast<int>(e % Dp);
    const float v = c < D ? rintf(src[e] - static_cast<float>(shift)) : 0.f;
    dst[e] = static_cast<int8_t>(fminf(fmaxf(v, -128.f), 127.f));
}

// the same rounding in fp32: rows of integers, each the value quantize_i8
// stores plus the shift (padding 0)
__global__ void round_to_int_kernel(const float* __restrict__ src, int64_t N, int D, int Dp, int shift,
                                    float* __restrict__ dst)
{
    const int64_t e = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (e >= N * Dp) return;
    const int c = static_cast<int>(e % Dp);
    const float v = c < D ? rintf(src[e] - static_cast<float>(shift)) : 0.f;
    dst[e] = c < D ? fminf(fmaxf(v, -128.f), 127.f) + static_cast<float>(shift) : 0.f;
}

// |x|^2 of int8 rows (exact integer sums), one wave per row
__global__ void __launch_bounds__(256) row_norms_i8_kernel(const int8_t* __restrict__ X, int64_t N, int Dp,
                                                           float* __restrict__ norms)
{
    const int64_t row = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (row >= N) return;
    int s = 0;
    for (int c = lane; c < Dp; c += 64) {
        const int v = X[row * Dp + c];
        s += v * v;
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) s += __shfl_xor(s, o);
    if (lane == 0) norms[row] = static_cast<float>(s);
}

// |x|^2 per row, one wave per row; summed in a fixed order.
__global__ void __launch_bounds__(256) row_norms_kernel(const float* __restrict__ X, int64_t N, int Dp,
                                                        float* __restrict__ norms)
{
    const int64_t row = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (row >= N) return;
    float s = 0.f;
    for (int c = lane; c < Dp; c += 64) {
        const float v = X[row * Dp + c];
        s = fmaf(v, v, s);
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) s += __shfl_xor(s, o);
    if (lane == 0) norms[row] = s;
}

// pool list of every bucket = concatenation of member ranges (copy tasks).
struct CopyTask { int64_t src; int64_t dst; int64_t n; };
__global__ void copy_ranges_kernel(const CopyTask* __restrict__ tasks, const int32_t* __restrict__ members,
                                   int32_t* __restrict__ pool)
{
    const CopyTask t = tasks[blockIdx.x];
    for (int64_t e = threadIdx.x; e < t.n; e += blockDim.x) pool[t.dst + e] = members[t.src + e];
}

__global__ void negate_kernel(float* __restrict__ d, int64_t n)
{
    const int64_t e = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (e < n) d[e] = -d[e];
}

// ------------------------------------------------------------------ sanitize
// src/optimize.cu:89-134: -1 / out-of-range / self -> first valid entry of the
// row, else (i+1) % N.  One wave per row.
__global__ void __launch_bounds__(256) sanitize_kernel(const int32_t* __restrict__ in, int64_t N, int M,
                                                       uint32_t* __restrict__ out)
{
    const int64_t i = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (i >= N) return;
    int first = INT_MAX;
    for (int k = lane; k < M; k += 64) {
        const int32_t v = in[i * M + k];
        if (v >= 0 && v < N && v != i) { first = k; break; }
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) first = min(first, __shfl_xor(first, o));
    const uint32_t fallback = first == INT_MAX ? static_cast<uint32_t>((i + 1) % N)
                                               : static_cast<uint32_t>(in[i * M + first]);
    for (int k = lane; k < M; k += 64) {
        const int32_t v = in[i * M + k];
        out[i * M + k] = (v < 0 || v >= N || v == i) ? fallback : static_cast<uint32_t>(v);
    }
}

// The same rule for M in {16, 32, 64, 128}: L = M / 4 lanes per row, each
// with one 16-byte load and store, 64 / L rows per wave, the row's first
// valid entry by a min over its lanes.
template <int L>
__global__ void __launch_bounds__(256) sanitize_vec_kernel(const int4* __restrict__ in, int64_t N,
                                                           uint4* __restrict__ out)
{
    constexpr int R = 64 / L;   // rows per wave
    const int lane = threadIdx.x & 63;
    const int64_t i = (static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6)) * R + lane / L;
    const int part = lane % L;
    const bool live = i < N;
    const int4 v = live ? in[i * L + part] : make_int4(-1, -1, -1, -1);
    const int32_t e[4] = {v.x, v.y, v.z, v.w};
    bool ok[4];
    int first = INT_MAX;
#pragma unroll
    for (int u = 3; u >= 0; --u) {
        ok[u] = e[u] >= 0 && e[u] < N && e[u] != i;
        if (ok[u]) first = 4 * part + u;
    }
#pragma unroll
    for (int o = 1; o < L; o <<= 1) first = min(first, __shfl_xor(first, o));
    // the row's first valid entry, from the lane that holds it
    const int src = (lane & ~(L - 1)) | ((first == INT_MAX ? 0 : first) >> 2);
    const int sel = (first == INT_MAX ? 0 : first) & 3;
    const int32_t mine = sel == 0 ? e[0] : sel == 1 ? e[1] : sel == 2 ? e[2] : e[3];
    const int32_t got = __shfl(mine, src);
    const uint32_t fb = first == INT_MAX ? static_cast<uint32_t>((i + 1) % N) : static_cast<uint32_t>(got);
    if (live)
        out[i * L + part] = make_uint4(ok[0] ? e[0] : fb, ok[1] ? e[1] : fb, ok[2] ? e[2] : fb, ok[3] ? e[3] : fb);
}

// ------------------------------------------------------------------ prune
// CAGRA detour-count prune of one point per wave.
// count[kAB] = #{kAD < kAB : D = row[kAD] in [0,N), row[kAB] in row(D)},
// each (kAD, kAB) once, duplicate ids of the row as separate ranks
// (src/prune_windowed_core.hpp:189-232); output = first K valid entries in
// (count, rank) order (src/prune_windowed_core.hpp:238-263).
constexpr int kPruneMaxM = 128;
constexpr int kPruneDepth = 8;    // neighbour rows in flight per wave

// One wave per point a.  Row a's ids go into an LDS hash table of 4-slot
// buckets (2*MM buckets; a full bucket spills into the next one, no
// wrap-around; a repeated id takes one slot per occurrence); each lane
// remembers the slots of its own entries.  Every neighbour row kAD < M-1 is
// then streamed through, kPruneDepth rows in flight: a lane whose id matches
// a slot (one 16-byte read per bucket probed) sets bit kAD - kd0 of that
// slot's 8-bit tag (kd0: the first row of the group of kPruneDepth rows; an
// id repeated in the neighbour row sets the same bit, so each (kAD, kAB) pair
// counts once); a bucket's four tags share one word.  After each group the
// lane owning rank kAB counts the bits of rows kAD < kAB in its slot's tag,
// and once every lane has read, the owners clear their words -- one tag read
// per group instead of one per row, and no wait between a row's tag writes
// and the next row's bucket reads (src/prune_windowed_core.hpp:177-232).
// Only slots that hold an id of row a are ever tagged, and each belongs to
// one lane, so the clears leave the whole tag array zero.  The counts stay in registers;
// the neighbour row's id is read from row a's registers by readlane, so its
// address is scalar work.  Finally the first K valid ranks by (count, rank)
// are written (src/prune_windowed_core.hpp:234-263).  E = list halves of 64.
// Home bucket of an id: a multiplicative hash on the id's low 24 bits
// (v_mul_u32_u24 issues at full rate, a 32-bit multiply at a quarter); ids
// that differ only above bit 23 share a home and spill, which costs probes,
// not results.
__device__ __forceinline__ uint32_t prune_hash(int32_t v, uint32_t mask)
{
    uint32_t p;
    // (the compiler would fold the 24-bit mask into the bit range it keeps
    // and pick the quarter-rate 32-bit multiply)
    asm("v_mul_u32_u24 %0, 0x9e3779, %1" : "=v"(p) : "v"(v));
    return (p >> 15) & mask;
}

// Last processing position p with off[p] <= id (positions 0 .. nb - 1).
__device__ __forceinline__ int prune_pos_of(const uint32_t* __restrict__ off, int nb, uint32_t id)
{
    int lo = 0, hi = nb - 1;
    while (lo < hi) {
        const int mid = (lo + hi + 1) >> 1;
        if (off[mid] <= id) lo = mid;
        else hi = mid - 1;
    }
    return lo;
}

// ROWS selects where the rows live:
//   0: the whole table, row r at G + r * M;
//   1: a chunk's rows and all their neighbours' rows in a compact table, row r
//      at G + map.cidx[r] * M (every row the chunk reads is loaded);
//   2: bucket windows (src/prune_windowed_gpu.cu:181-326 semantics): rows are
//      numbered by processing position, position q owning ids
//      [off[q], off[q + 1]); row a at position p may count detours only
//      through neighbours whose position is in p's window (win[p * W ..],
//      win_len[p] entries) and loaded (cbase[q] >= 0: the compact row of
//      off[q]); any other neighbour contributes nothing.
// ROWS 1 and 2 prune rows map.a0 .. map.a0 + map.n - 1 into output rows
// 0 .. n - 1.
// BUF (ROWS 0, tables below 4 GiB): neighbour rows by buffer loads, the
// row's byte offset a scalar operand of the load.
template <int E, int ROWS, bool BUF = false>
__global__ void __launch_bounds__(256) cagra_prune_kernel(const int32_t* __restrict__ G, int64_t N, int M, int K,
                                                          uint32_t* __restrict__ out,
                                                          unsigned long long* __restrict__ bad_row, PruneMap map)
{
    static_assert(!BUF || ROWS == 0, "buffer loads address the whole table");
    constexpr int MM = 64 * E;
    constexpr int NBK = 2 * MM;               // home buckets
    constexpr int BK = NBK + MM / 4 + 1;      // + spill room: at most MM entries
    constexpr int SLOTS = 4 * BK;
    constexpr uint32_t mask = NBK - 1;
    constexpr uint32_t kEmpty = 0xffffffffu;
    static_assert(kPruneDepth <= 8, "one tag bit per row of a group, 8-bit tags");
    constexpr int TAGW = BK + 16;             // + 64 never-tagged tags (invalid entries)
    __shared__ __align__(16) uint32_t tab[4][SLOTS];
    __shared__ uint32_t tag[4][TAGW];         // slot s: bits 8*(s%4).. of word s/4
    const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int64_t a0 = ROWS == 0 ? 0 : map.a0;
    int64_t a;
    if (ROWS == 0) {
        // block b takes positions 4 (x * per_xcd + b / 8) .. + 3 of the
        // order, x = b % 8 (per_xcd = gridDim.x / 8): the workgroups go
        // round-robin to the 8 XCDs, so each XCD walks its own contiguous
        // eighth of the order, and with the bucket order its L2 keeps the
        // neighbour rows of the bucket it is on
        const int64_t per_xcd = gridDim.x / 8;
        const int64_t q = (static_cast<int64_t>(blockIdx.x % 8) * per_xcd + blockIdx.x / 8) * 4 + w;
        if (q >= N) return;
        a = map.order ? map.order[q] : q;
    } else {
        a = a0 + static_cast<int64_t>(blockIdx.x) * 4 + w;
        if (a >= map.a0 + map.n) return;
    }
    int64_t arow = a;
    int pa = 0;
    if (ROWS == 1) arow = map.cidx[a];
    if (ROWS == 2) {
        pa = prune_pos_of(map.off, map.n_buckets, static_cast<uint32_t>(a));
        arow = map.cbase[pa] + (a - map.off[pa]);
    }

    // ids below nlim are rows of G (ROWS 0)
    const uint32_t nlim = static_cast<uint32_t>(min(N, static_cast<int64_t>(0x80000000u)));
    for (int s = lane; s < SLOTS; s += 64) tab[w][s] = kEmpty;
    for (int s = lane; s < TAGW; s += 64) tag[w][s] = 0u;
    int32_t A[E];
    int col[E];
#pragma unroll
    for (int e = 0; e < E; ++e) {
        const int k = lane + 64 * e;
        col[e] = k < M ? k : M - 1;
        A[e] = k < M ? G[arow * M + k] : -1;
    }
    // the row of each neighbour in G (-1: not to be read)
    int64_t nrow[E];
#pragma unroll
    for (int e = 0; ROWS != 0 && e < E; ++e) {
        const bool v = A[e] >= 0 && A[e] < N;
        nrow[e] = v ? static_cast<int64_t>(A[e]) : -1;
        if (ROWS == 1 && v) nrow[e] = map.cidx[A[e]];
        if (ROWS == 2 && v) {
            const int q = prune_pos_of(map.off, map.n_buckets, static_cast<uint32_t>(A[e]));
            const int32_t* wp = map.win + static_cast<int64_t>(pa) * map.W;
            const int wl = map.win_len[pa];
            bool inw = false;
            for (int i = 0; i < wl; ++i) inw |= wp[i] == q;
            const int64_t cb = map.cbase[q];
            nrow[e] = inw && cb >= 0 ? cb + (A[e] - static_cast<int64_t>(map.off[q])) : -1;
        }
    }
    wave_sync();
    // insertion; every entry ends up at most dmax buckets past its home
    int slot[E];
    uint32_t disp = 0;
#pragma unroll
    for (int e = 0; e < E; ++e) {
        slot[e] = SLOTS + lane;
        if (A[e] >= 0) {
            const uint32_t home = prune_hash(A[e], mask);
            uint32_t h = 4 * home;
            while (atomicCAS(&tab[w][h], kEmpty, static_cast<uint32_t>(A[e])) != kEmpty) ++h;
            slot[e] = static_cast<int>(h);
            disp = max(disp, h / 4 - home);
        }
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) disp = max(disp, static_cast<uint32_t>(__shfl_xor(static_cast<int>(disp), o)));
    const uint32_t dmax = static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<int>(disp)));
    wave_sync();

    // rows in flight: raw ids plus whether the row exists; the ids are
    // checked when the row is probed, so no load is waited for early
    int32_t ring[kPruneDepth][E];
    bool rok[kPruneDepth];
    // ROWS 0: row a's ids with the last rank and everything past it -1
    // (never fetched), so that a fetch needs no rank test
    int32_t Apad[E];
#pragma unroll
    for (int e = 0; e < E; ++e) Apad[e] = lane + 64 * e < M - 1 ? A[e] : -1;
    // (unused without BUF)
    const __amdgpu_buffer_rsrc_t grsrc = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<int32_t*>(G), 0, BUF ? static_cast<int>(N * M * 4) : 0, 0x00020000);
    auto fetch = [&](int kAD, int32_t (&b)[E], bool& ok) {
        if constexpr (ROWS == 0) {
            // the id (negative ids and the padding fail du < nlim) and the
            // row address stay on the scalar unit
            const int kk = min(kAD, MM - 1);
            uint32_t du = __builtin_amdgcn_readlane(static_cast<uint32_t>(Apad[0]), kk & 63);
            if constexpr (E > 1) {
                const uint32_t d1 = __builtin_amdgcn_readlane(static_cast<uint32_t>(Apad[E - 1]), kk & 63);
                du = (kk >> 6) ? d1 : du;
            }
            ok = du < nlim;
            if constexpr (BUF) {
                const uint32_t soff = ok ? du * static_cast<uint32_t>(4 * M) : 0u;
#pragma unroll
                for (int e = 0; e < E; ++e) b[e] = __builtin_amdgcn_raw_buffer_load_b32(grsrc, 4 * col[e], soff, 0);
            } else {
                const int32_t* row = G + static_cast<int64_t>(ok ? du : 0u) * M;
#pragma unroll
                for (int e = 0; e < E; ++e) b[e] = row[col[e]];
            }
            return;
        }
        int64_t d = -1;
        if (kAD < M - 1) {
#pragma unroll
            for (int e = 0; e < E; ++e)
                if ((kAD >> 6) == e) {
                    const uint32_t lo = __builtin_amdgcn_readlane(static_cast<uint32_t>(nrow[e]), kAD & 63);
                    const int32_t hi = __builtin_amdgcn_readlane(static_cast<int32_t>(nrow[e] >> 32), kAD & 63);
                    d = (static_cast<int64_t>(hi) << 32) | lo;
                }
        }
        ok = d >= 0;
        const int32_t* row = G + (ok ? d : int64_t(0)) * M;
#pragma unroll
        for (int e = 0; e < E; ++e) b[e] = row[col[e]];
    };
    uint32_t c[E];
#pragma unroll
    for (int e = 0; e < E; ++e) c[e] = 0;
    // bit `bit` of the tag of every slot of bucket x (at base) holding v (an
    // id repeated in row a has a slot per copy, all tagged); bit is a
    // constant of the unrolled row loop, so the word is four selects
    auto tag_bucket = [&](const uint4& x, uint32_t v, bool valid, uint32_t base, uint32_t bit) {
        const uint32_t t = (x.x == v ? bit : 0u) | (x.y == v ? bit << 8 : 0u) | (x.z == v ? bit << 16 : 0u) |
                           (x.w == v ? bit << 24 : 0u);
        if (valid && t != 0u) atomicOr(&tag[w][base / 4], t);
    };
    // rows kd0 .. kd0 + kPruneDepth - 1 of the ring (row kd0 + r in slot r);
    // each slot is refilled with row kd0 + r + kPruneDepth once probed
    auto probe_group = [&](int kd0) {
        if (dmax == 0) {
            // every entry sits in its home bucket: one bucket read per id
#pragma unroll
            for (int r = 0; r < kPruneDepth; ++r) {
#pragma unroll
                for (int e = 0; e < E; ++e) {
                    const uint32_t base = 4 * prune_hash(ring[r][e], mask);
                    const uint4 x = *reinterpret_cast<const uint4*>(&tab[w][base]);
                    if (rok[r])
                        tag_bucket(x, static_cast<uint32_t>(ring[r][e]), lane + 64 * e < M && ring[r][e] >= 0, base,
                                   1u << r);
                }
                fetch(kd0 + r + kPruneDepth, ring[r], rok[r]);
            }
        } else {
            // every occurrence of v in row a lies within dmax buckets of v's
            // home: a fixed, wave-uniform number of bucket reads
#pragma unroll
            for (int r = 0; r < kPruneDepth; ++r) {
                if (rok[r]) {
#pragma unroll
                    for (int e = 0; e < E; ++e) {
                        const uint32_t v = static_cast<uint32_t>(ring[r][e]);
                        const bool valid = lane + 64 * e < M && ring[r][e] >= 0;
                        const uint32_t home = prune_hash(ring[r][e], mask);
                        for (uint32_t s = 0; s <= dmax; ++s) {
                            const uint32_t base = 4 * (home + s);
                            tag_bucket(*reinterpret_cast<const uint4*>(&tab[w][base]), v, valid, base, 1u << r);
                        }
                    }
                }
                fetch(kd0 + r + kPruneDepth, ring[r], rok[r]);
            }
        }
        wave_sync();
        uint32_t t[E];
#pragma unroll
        for (int e = 0; e < E; ++e) t[e] = tag[w][slot[e] / 4];
        wave_sync();   // every tag word read before any is cleared
#pragma unroll
        for (int e = 0; e < E; ++e) {
            const uint32_t mine = (t[e] >> (8 * (slot[e] % 4))) & 0xffu;
            const int m = lane + 64 * e - kd0;   // rows kd0 + r < kAB count
            const uint32_t below = m <= 0 ? 0u : m >= 8 ? 0xffu : (1u << m) - 1u;
            c[e] += static_cast<uint32_t>(__popc(mine & below));
            tag[w][slot[e] / 4] = 0u;
        }
        wave_sync();
    };
#pragma unroll
    for (int r = 0; r < kPruneDepth; ++r) fetch(r, ring[r], rok[r]);
    for (int kd = 0; kd < M - 1; kd += kPruneDepth) probe_group(kd);

    int nvalid = 0;
#pragma unroll
    for (int e = 0; e < E; ++e) nvalid += __popcll(__ballot(A[e] >= 0));
    if (nvalid < K) {
        if (lane == 0) atomicMin(bad_row, static_cast<unsigned long long>(a));
        return;
    }
    const int64_t orow = a - a0;
    // position = valid entries before this one in (count, rank) order; one
    // key per entry, count << 8 | rank (counts < 128), invalid = all ones,
    // kept in the hash table's LDS (no longer read); fewer LDS bytes per
    // block let one more block share a CU
    uint32_t* skey = tab[w];
    uint32_t key[E];
#pragma unroll
    for (int e = 0; e < E; ++e) {
        key[e] = A[e] >= 0 ? (c[e] << 8) | static_cast<uint32_t>(lane + 64 * e) : 0xffffffffu;
        skey[lane + 64 * e] = key[e];
    }
    wave_sync();
    int pos[E];
#pragma unroll
    for (int e = 0; e < E; ++e) pos[e] = 0;
#pragma unroll 4
    for (int q4 = 0; q4 < MM / 4; ++q4) {
        const uint4 kq = *reinterpret_cast<const uint4*>(&skey[4 * q4]);
#pragma unroll
        for (int e = 0; e < E; ++e)
            pos[e] += (kq.x < key[e] ? 1 : 0) + (kq.y < key[e] ? 1 : 0) + (kq.z < key[e] ? 1 : 0) +
                      (kq.w < key[e] ? 1 : 0);
    }
#pragma unroll
    for (int e = 0; e < E; ++e)
        if (A[e] >= 0 && pos[e] < K) out[orow * K + pos[e]] = static_cast<uint32_t>(A[e]);
}

// ------------------------------------------------------------------ reverse merge
// Reverse edges {dst = fwd[i][k], src = i, rank = k} (src/optimize_chunked.cu:372-407)
// grouped per dst, ordered by (rank, src) (src/edge_chunk_accumulator.hpp:235-284),
// and merged into the dst's forward row with K/2 protected slots
// (src/edge_chunk_accumulator.hpp:471-494).

// In-degree of every node; each edge keeps the slot the count gave it inside
// its destination's segment (any slot order works: segments are re-ordered
// by the (rank, src) key before use).
__global__ void rev_count_kernel(const uint32_t* __restrict__ fwd, int64_t E, int64_t N, uint32_t* __restrict__ deg,
                                 uint32_t* __restrict__ slot, int* __restrict__ err)
{
    const int64_t e = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (e >= E) return;
    const uint32_t j = fwd[e];
    if (j >= N) { atomicExch(err, 1); return; }
    slot[e] = atomicAdd(&deg[j], 1u);
}

__global__ void rev_scatter_kernel(const uint32_t* __restrict__ fwd, int64_t E, int64_t N, int K,
                                   const uint32_t* __restrict__ off, const uint32_t* __restrict__ slot,
                                   unsigned long long* __restrict__ keys)
{
    const int64_t e = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (e >= E) return;
    const uint32_t j = fwd[e];
    if (j >= N) return;
    const int64_t i = e / K;
    const uint32_t k = static_cast<uint32_t>(e - i * K);
    keys[off[j] + slot[e]] = (static_cast<unsigned long long>(k) << 32) | static_cast<uint32_t>(i);
}

// Exclusive scan of n uint32 counts into out[0..n] (out[n] = total).
constexpr int kScanBlock = 1024;
__global__ void __launch_bounds__(256) scan_block_kernel(const uint32_t* __restrict__ in, int64_t n,
                                                         uint32_t* __restrict__ out, uint32_t* __restrict__ sums)
{
    __shared__ uint32_t s[256];
    const int64_t base = static_cast<int64_t>(blockIdx.x) * kScanBlock;
    uint32_t v[4];
    uint32_t local = 0;
#pragma unroll
    for (int u = 0; u < 4; ++u) {
        const int64_t e = base + threadIdx.x * 4 + u;
        v[u] = e < n ? in[e] : 0u;
        local += v[u];
    }
    s[threadIdx.x] = local;
    __syncthreads();
    for (int off = 1; off < 256; off <<= 1) {
        const uint32_t t = threadIdx.x >= off ? s[threadIdx.x - off] : 0u;
        __syncthreads();
        s[threadIdx.x] += t;
        __syncthreads();
    }
    uint32_t run = s[threadIdx.x] - local;
#pragma unroll
    for (int u = 0; u < 4; ++u) {
        const int64_t e = base + threadIdx.x * 4 + u;
        if (e < n) out[e] = run;
        run += v[u];
    }
    if (threadIdx.x == 255) sums[blockIdx.x] = s[255];
}

__global__ void __launch_bounds__(256) scan_sums_kernel(uint32_t* __restrict__ sums, int64_t nb,
                                                        uint32_t* __restrict__ total)
{
    __shared__ uint32_t s[256];
    uint32_t carry = 0;
    for (int64_t b0 = 0; b0 < nb; b0 += 256) {
        const int64_t e = b0 + threadIdx.x;
        const uint32_t v = e < nb ? sums[e] : 0u;
        s[threadIdx.x] = v;
        __syncthreads();
        for (int off = 1; off < 256; off <<= 1) {
            const uint32_t t = threadIdx.x >= off ? s[threadIdx.x - off] : 0u;
            __syncthreads();
            s[threadIdx.x] += t;
            __syncthreads();
        }
        if (e < nb) sums[e] = carry + s[threadIdx.x] - v;
        const uint32_t blk = s[255];
        __syncthreads();
        carry += blk;
    }
    if (threadIdx.x == 0) *total = carry;
}

__global__ void scan_add_kernel(uint32_t* __restrict__ out, int64_t n, const uint32_t* __restrict__ sums)
{
    const int64_t e = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (e < n) out[e] += sums[e / kScanBlock];
}

__device__ __forceinline__ unsigned long long wave_min_u64(unsigned long long v)
{
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        const unsigned long long t = __shfl_xor(v, o);
        v = t < v ? t : v;
    }
    return v;
}

// One dst row j, by one wave.  The final row is
//   protected S = fwd[j][0..P)  ++  R  ++  (O minus the first occurrence of each r in R)
// truncated to K, where O = fwd[j][P..K) and R = the distinct sources not in
// S, by strongest (rank, src) key, at most L = K-P of them.  This is the
// fixed point of the weakest-first move-to-front insertion of
// merge_rank_ordered_into_row (an accessed source moves to slot P; absent
// ones push the last slot out).  keys: the row's n reverse keys
// (rank << 32 | src) in any order; sR, sRow, sK: the wave's LDS scratch.
constexpr int kRevMaxK = 64;

// The global reads of one row, issued ahead of its merge: the forward row
// (one id per lane) and, for at most 64 keys, one key per lane.
struct RevRow {
    uint32_t rowv;
    unsigned long long key;
    const unsigned long long* keys;
    uint32_t n;
};

__device__ __forceinline__ RevRow rev_row_load(const uint32_t* __restrict__ fwd, int64_t j, int K,
                                               const unsigned long long* keys, uint32_t n, int lane)
{
    RevRow r;
    r.rowv = lane < K ? fwd[j * K + lane] : 0xffffffffu;
    r.key = n <= 64 && lane < static_cast<int>(n) ? keys[lane] : ~0ull;
    r.keys = keys;
    r.n = n;
    return r;
}

// v among a[lo, min(hi, lim)), a: 64 LDS words, 16-byte aligned; lo and hi
// wave-uniform (hi <= 64), lim per lane.  Reads go out 16 words at a time.
__device__ __forceinline__ bool lds_has(const uint32_t* a, int lo, int hi, int lim, uint32_t v)
{
    bool f = false;
    for (int b = lo & ~15; b < hi; b += 16) {
        uint4 x[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) x[u] = *reinterpret_cast<const uint4*>(a + b + 4 * u);
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const int i = b + 4 * u;
            const uint32_t e[4] = {x[u].x, x[u].y, x[u].z, x[u].w};
#pragma unroll
            for (int c = 0; c < 4; ++c) f |= i + c >= lo && i + c < hi && i + c < lim && e[c] == v;
        }
    }
    return f;
}

// Number of the first 2*npair entries of sK (64 keys, 16-byte aligned)
// below key; dup: one of those has src's id.  Eight keys per batch of reads.
__device__ __forceinline__ int keys_below(const unsigned long long* sK, int npair, unsigned long long key,
                                          uint32_t src, bool& dup)
{
    int pos = 0;
    bool d = false;
    for (int q = 0; q < npair; q += 4) {
        uint4 x[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) x[u] = *reinterpret_cast<const uint4*>(&sK[2 * (q + u)]);
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const unsigned long long k0 = (static_cast<unsigned long long>(x[u].y) << 32) | x[u].x;
            const unsigned long long k1 = (static_cast<unsigned long long>(x[u].w) << 32) | x[u].z;
            const bool l0 = k0 < key, l1 = k1 < key;
            pos += (l0 ? 1 : 0) + (l1 ? 1 : 0);
            d |= (l0 && x[u].x == src) || (l1 && x[u].z == src);
        }
    }
    dup = d;
    return pos;
}

__device__ __forceinline__ void rev_merge_row(const RevRow& in, int64_t j, int K, uint32_t* __restrict__ out,
                                              uint32_t* sR, uint32_t* sRow, unsigned long long* sK, int lane)
{
    const int P = K / 2, L = K - P;
    const uint32_t rowv = in.rowv;
    const uint32_t n = in.n;
    const unsigned long long* keys = in.keys;
    const unsigned long long below = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
    wave_sync();   // the wave's previous row is done with the scratch
    sRow[lane] = rowv;
    wave_sync();
    int nR = 0;

    // s among the protected slots fwd[j][0..P) (LDS broadcast reads)
    auto protected_src = [&](uint32_t s) { return lds_has(sRow, 0, P, 64, s); };

    if (n <= 64) {
        // R by counting: protected sources drop out first; a key's position
        // is the number of smaller remaining keys.  A source repeated in the
        // keys keeps only its strongest key (then the positions are counted
        // again without the weaker copies).
        unsigned long long key = in.key;
        const uint32_t src = static_cast<uint32_t>(key);
        if (key != ~0ull && protected_src(src)) key = ~0ull;
        sK[lane] = key;
        wave_sync();
        const int npair = static_cast<int>(n + 1) / 2;
        bool dup = false;
        int pos = keys_below(sK, npair, key, src, dup);
        bool keep = key != ~0ull;
        if (__ballot(keep && dup)) {
            keep = keep && !dup;
            wave_sync();
            sK[lane] = keep ? key : ~0ull;
            wave_sync();
            bool unused = false;
            pos = keys_below(sK, npair, key, src, unused);
        }
        if (keep && pos < L) sR[pos] = src;
        nR = min(L, static_cast<int>(__popcll(__ballot(keep))));
    } else {
        // long lists, 64 keys at a time: the best L keys so far stay sorted
        // in sB (over sR's memory); a chunk's keys below the L-th best are
        // ranked against them and against each other
        unsigned long long* sB = reinterpret_cast<unsigned long long*>(sR);
        if (lane < 32) sB[lane] = ~0ull;
        int nb = 0;
        unsigned long long thr = ~0ull;
        for (uint32_t c = 0; c < n; c += 64) {
            const unsigned long long key = c + lane < n ? keys[c + lane] : ~0ull;
            bool cand = key < thr;
            if (cand) cand = !protected_src(static_cast<uint32_t>(key));
            const unsigned long long cm = __ballot(cand);
            if (cm == 0) continue;
            const int nc = static_cast<int>(__popcll(cm));
            wave_sync();
            if (cand) sK[__popcll(cm & below)] = key;
            wave_sync();
            const unsigned long long mc = lane < nc ? sK[lane] : ~0ull;
            const unsigned long long mb = lane < nb ? sB[lane] : ~0ull;
            int pc = 0, pb = lane;
            for (int q = 0; q < nc; ++q) {
                const unsigned long long x = sK[q];
                pc += x < mc ? 1 : 0;
                pb += x < mb ? 1 : 0;
            }
            for (int q = 0; q < nb; ++q) pc += sB[q] < mc ? 1 : 0;
            wave_sync();
            if (lane < nb && pb < L) sB[pb] = mb;
            if (lane < nc && pc < L) sB[pc] = mc;
            nb = min(L, nb + nc);
            wave_sync();
            thr = nb == L ? sB[L - 1] : ~0ull;
        }
        // a source twice among the chosen keys (a forward row that repeats
        // an id): the exact scan below decides instead
        wave_sync();
        const unsigned long long mb = lane < nb ? sB[lane] : ~0ull;
        bool dupb = false;
        for (int q = 0; q < nb; ++q) {
            const unsigned long long x = sB[q];
            dupb |= x < mb && static_cast<uint32_t>(x) == static_cast<uint32_t>(mb);
        }
        const bool any_dup = __ballot(dupb) != 0;
        wave_sync();
        if (!any_dup) {
            if (lane < nb) sR[lane] = static_cast<uint32_t>(mb);
            nR = nb;
        } else {
            // the strongest remaining key by wave minimum, L times
            unsigned long long last = 0;
            bool first = true;
            while (nR < L) {
                unsigned long long m = ~0ull;
                for (uint32_t e = lane; e < n; e += 64) {
                    const unsigned long long v = keys[e];
                    if ((first || v > last) && v < m) m = v;
                }
                m = wave_min_u64(m);
                if (m == ~0ull) break;
                first = false;
                last = m;
                const uint32_t src = static_cast<uint32_t>(m);
                bool skip = protected_src(src);
                for (int q = 0; q < nR; ++q) skip |= (sR[q] == src);
                if (!skip) {
                    if (lane == 0) sR[nR] = src;
                    wave_sync();
                    ++nR;
                }
            }
        }
    }
    wave_sync();

    if (lane < P) out[j * K + lane] = rowv;
    if (lane < nR) out[j * K + P + lane] = sR[lane];
    if (nR < L) {
        // O entries, in order, minus the first occurrence of each element of R
        const bool inR = lds_has(sR, 0, nR, 64, rowv);
        const bool earlier = lds_has(sRow, P, K, lane, rowv);
        const bool consumed = inR && !earlier;
        const bool keepO = lane >= P && lane < K && !consumed;
        const unsigned long long km = __ballot(keepO);
        const int pos = P + nR + __popcll(km & below);
        if (keepO && pos < K) out[j * K + pos] = rowv;
    }
}

// Rows grouped through a CSR built with global atomics (rev_count/scatter):
// the path for graphs beyond the binned path's size limit.
__global__ void __launch_bounds__(256) rev_merge_kernel(const uint32_t* __restrict__ fwd, int64_t N, int K,
                                                        const uint32_t* __restrict__ off,
                                                        const unsigned long long* __restrict__ keys,
                                                        uint32_t* __restrict__ out)
{
    __shared__ __align__(16) uint32_t sR[4][kRevMaxK];
    __shared__ __align__(16) uint32_t sRow[4][kRevMaxK];
    __shared__ __align__(16) unsigned long long sK[4][64];
    const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int64_t j = static_cast<int64_t>(blockIdx.x) * 4 + w;
    if (j >= N) return;
    const uint32_t lo = off[j];
    const RevRow in = rev_row_load(fwd, j, K, keys + lo, off[j + 1] - lo, lane);
    rev_merge_row(in, j, K, out, sR[w], sRow[w], sK[w], lane);
}

// Binned reverse merge (no global atomics).  Rows are cut into bins of
// 2^shift consecutive dst ids.  (1) every block of edges counts its edges per
// bin in LDS; (2) an exclusive scan of the counts in (bin, block) order gives
// every (bin, block) pair its output range; (3) every block scatters its
// edges through LDS cursors, as (dst within bin << 40 | rank << 32 | src);
// (4) one workgroup per bin groups its keys by dst (LDS counting sort into a
// second buffer) and merges each of its rows.  The key order inside a row is
// irrelevant to rev_merge_row, so the result equals the CSR path's.
constexpr int kRevBinThreads = 512;
constexpr int kRevMaxBins = 16384;      // (1)-(3): one LDS counter per bin
constexpr int kRevMaxBinShift = 12;     // (4): rows per bin <= 4096

__global__ void __launch_bounds__(kRevBinThreads) rev_bin_count_kernel(const uint32_t* __restrict__ fwd, int64_t E,
                                                                       int64_t N, int64_t chunk, int shift, int nbins,
                                                                       uint32_t* __restrict__ hist,
                                                                       int* __restrict__ err)
{
    extern __shared__ uint32_t h[];   // nbins counters
    for (int i = threadIdx.x; i < nbins; i += kRevBinThreads) h[i] = 0u;
    __syncthreads();
    const int64_t e0 = static_cast<int64_t>(blockIdx.x) * chunk, e1 = min(E, e0 + chunk);
    bool bad = false;
    for (int64_t e = e0 + threadIdx.x; e < e1; e += 4 * kRevBinThreads) {
        uint32_t v[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const int64_t x = e + u * kRevBinThreads;
            v[u] = x < e1 ? fwd[x] : 0xffffffffu;
        }
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            if (e + u * kRevBinThreads >= e1) continue;
            if (v[u] >= N) bad = true;
            else atomicAdd(&h[v[u] >> shift], 1u);
        }
    }
    if (bad) atomicExch(err, 1);
    __syncthreads();
    for (int i = threadIdx.x; i < nbins; i += kRevBinThreads)
        hist[static_cast<int64_t>(i) * gridDim.x + blockIdx.x] = h[i];
}

__global__ void __launch_bounds__(kRevBinThreads) rev_bin_scatter_kernel(const uint32_t* __restrict__ fwd, int64_t E,
                                                                         int64_t N, int K, int64_t chunk, int shift,
                                                                         int nbins, const uint32_t* __restrict__ offs,
                                                                         unsigned long long* __restrict__ part)
{
    extern __shared__ uint32_t cur[];   // nbins cursors
    for (int i = threadIdx.x; i < nbins; i += kRevBinThreads)
        cur[i] = offs[static_cast<int64_t>(i) * gridDim.x + blockIdx.x];
    __syncthreads();
    const int64_t e0 = static_cast<int64_t>(blockIdx.x) * chunk, e1 = min(E, e0 + chunk);
    const uint32_t mask = (1u << shift) - 1u;
    const uint32_t uK = static_cast<uint32_t>(K);
    for (int64_t e = e0 + threadIdx.x; e < e1; e += 4 * kRevBinThreads) {
        uint32_t v[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const int64_t x = e + u * kRevBinThreads;
            v[u] = x < e1 ? fwd[x] : 0xffffffffu;
        }
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            if (v[u] >= N) continue;   // also the lanes past e1
            const uint32_t eu = static_cast<uint32_t>(e + u * kRevBinThreads);   // E < 2^32
            const uint32_t i = eu / uK, k = eu - i * uK;
            const uint32_t slot = atomicAdd(&cur[v[u] >> shift], 1u);
            part[slot] = (static_cast<unsigned long long>(v[u] & mask) << 40) |
                         (static_cast<unsigned long long>(k) << 32) | i;
        }
    }
}

__global__ void __launch_bounds__(kRevBinThreads) rev_bin_merge_kernel(const uint32_t* __restrict__ fwd, int64_t N,
                                                                       int K, int shift, int nblk,
                                                                       const uint32_t* __restrict__ offs,
                                                                       const unsigned long long* __restrict__ part,
                                                                       unsigned long long* __restrict__ grouped,
                                                                       uint32_t* __restrict__ out)
{
    constexpr int kW = kRevBinThreads / 64;
    constexpr int kU = 4;   // keys in flight per thread while grouping
    extern __shared__ uint32_t dyn[];   // start[2^shift + 1], cur[2^shift]
    __shared__ uint32_t wtot[kW + 1];
    __shared__ __align__(16) uint32_t sR[kW][kRevMaxK];
    __shared__ __align__(16) uint32_t sRow[kW][kRevMaxK];
    __shared__ __align__(16) unsigned long long sK[kW][64];
    uint32_t* start = dyn;
    uint32_t* cur = dyn + (1 << shift) + 1;
    const int t = threadIdx.x, w = t >> 6, lane = t & 63;
    const int64_t j0 = static_cast<int64_t>(blockIdx.x) << shift;
    const int rows = static_cast<int>(min<int64_t>(int64_t(1) << shift, N - j0));
    const uint32_t lo = offs[static_cast<int64_t>(blockIdx.x) * nblk];
    const uint32_t hi = offs[static_cast<int64_t>(blockIdx.x + 1) * nblk];
    for (int r = t; r < rows; r += kRevBinThreads) cur[r] = 0u;
    __syncthreads();
    for (uint32_t e = lo + t; e < hi; e += kU * kRevBinThreads) {
        unsigned long long k[kU];
#pragma unroll
        for (int u = 0; u < kU; ++u) k[u] = e + u * kRevBinThreads < hi ? part[e + u * kRevBinThreads] : ~0ull;
#pragma unroll
        for (int u = 0; u < kU; ++u)
            if (k[u] != ~0ull) atomicAdd(&cur[static_cast<uint32_t>(k[u] >> 40)], 1u);
    }
    __syncthreads();

    // exclusive scan of the row counts: per thread a run of rows, then the
    // runs' totals by wave scans
    const int per = (rows + kRevBinThreads - 1) / kRevBinThreads;
    const int r0 = t * per;
    uint32_t loc = 0;
    for (int q = 0; q < per; ++q)
        if (r0 + q < rows) loc += cur[r0 + q];
    uint32_t inc = loc;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const uint32_t x = __shfl_up(inc, o);
        if (lane >= o) inc += x;
    }
    if (lane == 63) wtot[w] = inc;
    __syncthreads();
    if (t == 0) {
        uint32_t run = 0;
        for (int q = 0; q < kW; ++q) {
            const uint32_t v = wtot[q];
            wtot[q] = run;
            run += v;
        }
        wtot[kW] = run;
    }
    __syncthreads();
    uint32_t run = wtot[w] + inc - loc;
    for (int q = 0; q < per; ++q)
        if (r0 + q < rows) {
            const uint32_t c = cur[r0 + q];
            start[r0 + q] = run;
            cur[r0 + q] = run;
            run += c;
        }
    if (t == 0) start[rows] = wtot[kW];
    __syncthreads();

    for (uint32_t e = lo + t; e < hi; e += kU * kRevBinThreads) {
        unsigned long long k[kU];
#pragma unroll
        for (int u = 0; u < kU; ++u) k[u] = e + u * kRevBinThreads < hi ? part[e + u * kRevBinThreads] : ~0ull;
#pragma unroll
        for (int u = 0; u < kU; ++u)
            if (k[u] != ~0ull) {
                const uint32_t slot = atomicAdd(&cur[static_cast<uint32_t>(k[u] >> 40)], 1u);
                grouped[lo + slot] = k[u] & 0xFFFFFFFFFFull;
            }
    }
    __syncthreads();   // the block's own global writes are visible to the block after the barrier
    // one wave per row, the next row's reads in flight during each merge
    int r = w;
    if (r >= rows) return;
    RevRow nxt = rev_row_load(fwd, j0 + r, K, grouped + lo + start[r], start[r + 1] - start[r], lane);
    for (; r < rows; r += kW) {
        const RevRow in = nxt;
        const int rn = r + kW;
        if (rn < rows) nxt = rev_row_load(fwd, j0 + rn, K, grouped + lo + start[rn], start[rn + 1] - start[rn], lane);
        rev_merge_row(in, j0 + r, K, out, sR[w], sRow[w], sK[w], lane);
    }
}

// ------------------------------------------------------------------ cross-round merge
// top-M by (distance, id) of run U new, an id of new already present in run
// dropped (src/bucket.cu:5021-5053, ties by id).  One wave per row, each wave
// taking rows gridDim.x * 4 apart with the next row's four input rows loaded
// while it merges the current one; both inputs ascending with (-1, +inf)
// padding at the end.
constexpr int kMergeMaxM = 128;
constexpr int kMergeBlocks = 2048;   // 8 blocks of 4 waves per CU
__global__ void __launch_bounds__(256) merge_rounds_kernel(const int32_t* __restrict__ ri, const float* __restrict__ rd,
                                                           const int32_t* __restrict__ ni, const float* __restrict__ nd,
                                                           int64_t N, int M, int32_t* __restrict__ oi,
                                                           float* __restrict__ od)
{
    __shared__ float sRd[4][kMergeMaxM], sNd[4][kMergeMaxM];
    __shared__ int32_t sRi[4][kMergeMaxM], sNi[4][kMergeMaxM];
    const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int64_t stride = static_cast<int64_t>(gridDim.x) * 4;
    int64_t row = static_cast<int64_t>(blockIdx.x) * 4 + w;
    if (row >= N) return;
    struct In {
        float rd[2], nd[2];
        int32_t ri[2], ni[2];
    };
    // a row's inputs (distances loaded with the ids, masked after)
    auto load = [&](int64_t r, In& x) {
#pragma unroll
        for (int e = 0; e < 2; ++e) {
            const int k = lane + 64 * e;
            const bool in = k < M;
            x.ri[e] = in ? ri[r * M + k] : -1;
            x.rd[e] = in ? rd[r * M + k] : INFINITY;
            x.ni[e] = in ? ni[r * M + k] : -1;
            x.nd[e] = in ? nd[r * M + k] : INFINITY;
        }
    };
    In cur;
    load(row, cur);
    for (; row < N; row += stride) {
        In nxt;
        if (row + stride < N) load(row + stride, nxt);
        float rdv[2], ndv[2];
        int32_t riv[2], niv[2];
        int nr = 0;
#pragma unroll
        for (int e = 0; e < 2; ++e) {
            const int k = lane + 64 * e;
            riv[e] = cur.ri[e];
            rdv[e] = riv[e] >= 0 ? cur.rd[e] : INFINITY;
            niv[e] = cur.ni[e];
            ndv[e] = niv[e] >= 0 ? cur.nd[e] : INFINITY;
            if (riv[e] < 0) riv[e] = INT_MAX;
            if (k < kMergeMaxM) { sRd[w][k] = rdv[e]; sRi[w][k] = riv[e]; }
            nr += __popcll(__ballot(riv[e] != INT_MAX));
        }
        wave_sync();
        // drop new ids already in run; compact the survivors (order preserved)
        bool keep[2];
#pragma unroll
        for (int e = 0; e < 2; ++e) {
            bool dup = false;
            if (niv[e] >= 0)
                for (int q = 0; q < nr; ++q) dup |= (sRi[w][q] == niv[e]);
            keep[e] = niv[e] >= 0 && !dup;
        }
        const unsigned long long below = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
        const unsigned long long k0 = __ballot(keep[0]), k1 = __ballot(keep[1]);
        const int c0 = static_cast<int>(__popcll(k0));
        const int nn = c0 + static_cast<int>(__popcll(k1));
        const int cidx[2] = {static_cast<int>(__popcll(k0 & below)), c0 + static_cast<int>(__popcll(k1 & below))};
#pragma unroll
        for (int e = 0; e < 2; ++e)
            if (keep[e]) { sNd[w][cidx[e]] = ndv[e]; sNi[w][cidx[e]] = niv[e]; }
        wave_sync();
#pragma unroll
        for (int e = 0; e < 2; ++e) {
            const int k = lane + 64 * e;
            if (k < nr) {
                const int pos = k + lower_bound_g(sNd[w], sNi[w], nn, rdv[e], riv[e]);
                if (pos < M) { oi[row * M + pos] = riv[e]; od[row * M + pos] = rdv[e]; }
            }
            if (keep[e]) {
                const int pos = cidx[e] + lower_bound_g(sRd[w], sRi[w], nr, ndv[e], niv[e]);
                if (pos < M) { oi[row * M + pos] = niv[e]; od[row * M + pos] = ndv[e]; }
            }
        }
        for (int p = nr + nn + lane; p < M; p += 64) { oi[row * M + p] = -1; od[row * M + p] = INFINITY; }
        wave_sync();   // the lists are read before the next row overwrites them
        cur = nxt;
    }
}

// ------------------------------------------------------------------ translate
// final[inv[i]][k] = inv[g[i][k]] (src/translate_graph_ids.hpp:75); rows hit
// are counted so the caller can check inv is a permutation.
__global__ void translate_kernel(const uint32_t* __restrict__ g, const uint32_t* __restrict__ inv, int64_t N, int K,
                                 uint32_t* __restrict__ out, uint32_t* __restrict__ hits, int* __restrict__ err)
{
    const int64_t e = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (e >= N * K) return;
    const int64_t i = e / K;
    const int k = static_cast<int>(e - i * K);
    const uint32_t r = inv[i];
    const uint32_t v = g[e];
    if (r >= N || v >= N) { atomicExch(err, 1); return; }
    out[static_cast<int64_t>(r) * K + k] = inv[v];
    if (k == 0) atomicAdd(&hits[r], 1u);
}

__global__ void check_hits_kernel(const uint32_t* __restrict__ hits, int64_t N, int* __restrict__ err)
{
    const int64_t e = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (e < N && hits[e] != 1u) atomicExch(err, 1);
}

// ------------------------------------------------------------------ reorder
//
// Reordered dataset: out row n = in row inv[n] (bucket-contiguous new ids,
// src/bucket.cu:9253-9400).  One wave per row, 16-byte words when the row
// length allows, else 4-byte words, else bytes.
template <typename W>
__global__ void __launch_bounds__(256) permute_rows_kernel(const W* __restrict__ in, const uint32_t* __restrict__ inv,
                                                           int64_t N, int64_t words, W* __restrict__ out)
{
    const int64_t row = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (row >= N) return;
    const uint32_t src = inv[row];
    if (src >= static_cast<uint64_t>(N)) return;   // rejected by the permutation check
    const W* a = in + static_cast<int64_t>(src) * words;
    W* b = out + row * words;
    for (int64_t k = lane; k < words; k += 64) b[k] = a[k];
}

// perm[inv[n]] = n, counting hits so that a non-permutation is reported
__global__ void invert_perm_kernel(const uint32_t* __restrict__ inv, int64_t N, uint32_t* __restrict__ perm,
                                   uint32_t* __restrict__ hits, int* __restrict__ err)
{
    const int64_t n = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (n >= N) return;
    const uint32_t r = inv[n];
    if (r >= static_cast<uint64_t>(N)) { atomicExch(err, 1); return; }
    perm[r] = static_cast<uint32_t>(n);
    atomicAdd(&hits[r], 1u);
}

// Table in new ids: out[n][k] = perm[ids[inv[n]][k]], -1 (any id outside
// [0, N)) kept as -1.
__global__ void remap_table_kernel(const int32_t* __restrict__ ids, const uint32_t* __restrict__ inv,
                                   const uint32_t* __restrict__ perm, int64_t N, int M, int32_t* __restrict__ out)
{
    const int64_t e = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (e >= N * M) return;
    const int64_t n = e / M;
    const int k = static_cast<int>(e - n * M);
    const uint32_t src = inv[n];
    if (src >= static_cast<uint64_t>(N)) return;
    const int32_t v = ids[static_cast<int64_t>(src) * M + k];
    out[e] = (v >= 0 && v < N) ? static_cast<int32_t>(perm[v]) : -1;
}

// ------------------------------------------------------------------ launchers

static unsigned grid_for(int64_t n, int per_block)
{
    return static_cast<unsigned>((n + per_block - 1) / per_block);
}

void launch_pad_convert(const void* src, int dtype, float* dst, int64_t N, int D, int Dp, hipStream_t s)
{
    const int64_t total = N * Dp;
    const unsigned grid = static_cast<unsigned>(std::min<int64_t>((total + 255) / 256, 65536));
    if (total == 0) return;
    if (dtype == 0)
        hipLaunchKernelGGL(pad_convert_kernel<float>, dim3(grid), dim3(256), 0, s, static_cast<const float*>(src), dst, N, D, Dp);
    else if (dtype == 1)
        hipLaunchKernelGGL(pad_convert_kernel<uint8_t>, dim3(grid), dim3(256), 0, s, static_cast<const uint8_t*>(src), dst, N, D, Dp);
    else
        hipLaunchKernelGGL(pad_convert_kernel<int8_t>, dim3(grid), dim3(256), 0, s, static_cast<const int8_t*>(src), dst, N, D, Dp);
    GT_HIP(hipGetLastError());
}

void launch_prepare_int(const void* src, int dtype, int64_t N, int D, int Dp, float* xf, float* nf, int8_t* x8,
                        float* n8, hipStream_t s)
{
    GT_REQUIRE((dtype == 1 || dtype == 2) && D >= 1 && D <= Dp && Dp <= 256 && Dp % 4 == 0,
               "integer rows of at most 256 columns");
    if (N <= 0) return;
    int lg = 0;
    while ((1 << lg) < Dp / 4) ++lg;
    const int64_t threads = N << lg;
    const unsigned grid = static_cast<unsigned>((threads + 255) / 256);
    const bool vec = D % 4 == 0 && (reinterpret_cast<uintptr_t>(src) & 3) == 0;
    if (dtype == 1) {
        const uint8_t* p = static_cast<const uint8_t*>(src);
        if (vec) hipLaunchKernelGGL((prepare_int_kernel<uint8_t, true>), dim3(grid), dim3(256), 0, s, p, N, D, Dp, 128, lg, xf, nf, x8, n8);
        else hipLaunchKernelGGL((prepare_int_kernel<uint8_t, false>), dim3(grid), dim3(256), 0, s, p, N, D, Dp, 128, lg, xf, nf, x8, n8);
    } else {
        const int8_t* p = static_cast<const int8_t*>(src);
        if (vec) hipLaunchKernelGGL((prepare_int_kernel<int8_t, true>), dim3(grid), dim3(256), 0, s, p, N, D, Dp, 0, lg, xf, nf, x8, n8);
        else hipLaunchKernelGGL((prepare_int_kernel<int8_t, false>), dim3(grid), dim3(256), 0, s, p, N, D, Dp, 0, lg, xf, nf, x8, n8);
    }
    GT_HIP(hipGetLastError());
}

void launch_pad_i8(const void* src, int dtype, int8_t* dst, int64_t N, int D, int Dp, hipStream_t s)
{
    const int64_t total = N * Dp;
    const unsigned grid = static_cast<unsigned>(std::min<int64_t>((total + 255) / 256, 65536));
    if (total == 0) return;
    if (dtype == 1)
        hipLaunchKernelGGL(pad_i8_kernel<uint8_t>, dim3(grid), dim3(256), 0, s, static_cast<const uint8_t*>(src), dst, N, D, Dp, 128);
    else
        hipLaunchKernelGGL(pad_i8_kernel<int8_t>, dim3(grid), dim3(256), 0, s, static_cast<const int8_t*>(src), dst, N, D, Dp, 0);
    GT_HIP(hipGetLastError());
}

// Counting sort of each segment [off[g], off[g+1]) of members by key
// (keys < 1024), one workgroup per segment; segments shorter than min_n are
// copied unchanged.  The order inside a key is not fixed.
__global__ void __launch_bounds__(256) segment_sort_kernel(const int32_t* __restrict__ members,
                                                           const int32_t* __restrict__ key,
                                                           const int64_t* __restrict__ off, int min_n,
                                                           const int32_t* __restrict__ remap,
                                                           const int64_t* __restrict__ remap_base,
                                                           int32_t* __restrict__ out)
{
    constexpr int kKeys = 1024;
    __shared__ uint32_t cnt[kKeys];
    __shared__ uint32_t wsum[4];
    const int64_t lo = off[blockIdx.x], hi = off[blockIdx.x + 1];
    const int t = threadIdx.x;
    if (hi - lo < min_n) {
        for (int64_t e = lo + t; e < hi; e += 256) out[e] = members[e];
        return;
    }
    // keys through the segment's remap table when there is one
    const int32_t* rm = remap ? remap + remap_base[blockIdx.x] : nullptr;
    auto key_of = [&](int64_t e) -> uint32_t {
        const uint32_t k = static_cast<uint32_t>(key[e]) & (kKeys - 1);
        return rm ? static_cast<uint32_t>(rm[k]) & (kKeys - 1) : k;
    };
    for (int k = t; k < kKeys; k += 256) cnt[k] = 0u;
    __syncthreads();
    for (int64_t e = lo + t; e < hi; e += 256) atomicAdd(&cnt[key_of(e)], 1u);
    __syncthreads();
    // exclusive scan: 4 counters per thread, then the 256 partial sums
    uint32_t v[4], loc = 0;
#pragma unroll
    for (int u = 0; u < 4; ++u) { v[u] = cnt[4 * t + u]; loc += v[u]; }
    const int lane = t & 63, w = t >> 6;
    uint32_t inc = loc;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const uint32_t x = __shfl_up(inc, o);
        if (lane >= o) inc += x;
    }
    if (lane == 63) wsum[w] = inc;
    __syncthreads();
    uint32_t base = 0;
    for (int q = 0; q < w; ++q) base += wsum[q];
    uint32_t run = base + inc - loc;
#pragma unroll
    for (int u = 0; u < 4; ++u) { cnt[4 * t + u] = run; run += v[u]; }
    __syncthreads();
    for (int64_t e = lo + t; e < hi; e += 256) {
        const uint32_t slot = atomicAdd(&cnt[key_of(e)], 1u);
        out[lo + slot] = members[e];
    }
}

// A greedy nearest-neighbour chain through each segment's sub-centroids:
// start at sub-centroid 0, step to the first unvisited one of the current
// one's neighbour list (nn: K entries per sub-centroid, positions within the
// segment, -1 padded), else to the smallest unvisited one.  pos[base + i] =
// place of sub-centroid i on the chain.  One wave per segment; lane 0 walks.
constexpr int kSubChainLds = 1024 * 9;   // neighbour ids of a bucket's sub-centroids held in LDS
__global__ void __launch_bounds__(64) sub_chain_kernel(const int32_t* __restrict__ nn, int K,
                                                       const int64_t* __restrict__ base,
                                                       const int32_t* __restrict__ count, int32_t* __restrict__ pos)
{
    __shared__ uint32_t seen[32];   // up to 1024 sub-centroids
    __shared__ int32_t tbl[kSubChainLds];
    const int g = blockIdx.x, lane = threadIdx.x;
    const int n = count[g];
    if (n <= 0) return;
    const int64_t b0 = base[g];
    // the bucket's neighbour lists go to LDS first (the walk reads them one
    // step after another)
    const bool in_lds = n * K <= kSubChainLds;
    if (in_lds)
        for (int e = lane; e < n * K; e += 64) tbl[e] = nn[b0 * K + e];
    if (lane < 32) seen[lane] = 0u;
    __syncthreads();
    // the whole wave takes each step: lanes < K test the K neighbours (the
    // first unseen in list order wins), else lanes < 32 test a word of the
    // seen bits each (the lowest unseen sub-centroid wins)
    int cur = 0;
    for (int step = 0; step < n; ++step) {
        if (lane == 0) {
            seen[cur >> 5] |= 1u << (cur & 31);
            pos[b0 + cur] = step;
        }
        wave_sync();
        int v = -1;
        bool ok = false;
        if (lane < K) {
            v = in_lds ? tbl[cur * K + lane] : nn[(b0 + cur) * K + lane];
            ok = v >= 0 && v < n && !((seen[v >> 5] >> (v & 31)) & 1u);
        }
        const uint64_t m = __ballot(ok);
        if (m) {
            cur = __shfl(v, __ffsll(static_cast<unsigned long long>(m)) - 1);
            continue;
        }
        uint32_t fr = 0u;
        if (lane < 32 && lane * 32 < n) {
            const int left = n - lane * 32;
            fr = ~seen[lane] & (left >= 32 ? ~0u : ((1u << left) - 1u));
        }
        const uint64_t fm = __ballot(fr != 0u);
        if (!fm) break;
        const int wl = __ffsll(static_cast<unsigned long long>(fm)) - 1;
        cur = wl * 32 + __ffs(__shfl(fr, wl)) - 1;
    }
}

void launch_segment_sort(const int32_t* members, const int32_t* key, const int64_t* off, int64_t nseg, int min_n,
                         const int32_t* remap, const int64_t* remap_base, int32_t* out, hipStream_t s)
{
    if (nseg <= 0) return;
    hipLaunchKernelGGL(segment_sort_kernel, dim3(static_cast<unsigned>(nseg)), dim3(256), 0, s, members, key, off,
                       min_n, remap, remap_base, out);
    GT_HIP(hipGetLastError());
}

void launch_sub_chain(const int32_t* nn, int K, const int64_t* base, const int32_t* count, int64_t nseg, int32_t* pos,
                      hipStream_t s)
{
    if (nseg <= 0) return;
    GT_REQUIRE(K >= 1 && K <= 64, "sub-centroid chain: 1..64 neighbours (one lane each)");
    hipLaunchKernelGGL(sub_chain_kernel, dim3(static_cast<unsigned>(nseg)), dim3(64), 0, s, nn, K, base, count, pos);
    GT_HIP(hipGetLastError());
}

// Row norms (the order of row_norms_kernel, so the same bits) plus, per
// block of kNrBlockRows rows, whether every value is an integer and their
// range: part[3b] = 1 on a non-integer / non-finite value, part[3b+1] /
// part[3b+2] = min / max as ints; int_range_final_kernel folds the blocks
// into out[3].  Each wave takes kNrBlockRows / 4 rows, kNrGroup at a time
// with all their loads issued together.
constexpr int kNrBlockRows = 64;
constexpr int kNrGroup = 8;
__global__ void __launch_bounds__(256) row_norms_range_kernel(const float* __restrict__ X, int64_t N, int Dp,
                                                              float* __restrict__ norms, int* __restrict__ part)
{
    __shared__ int red[4][3];
    const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
    constexpr int WR = kNrBlockRows / 4;
    const int64_t r0 = static_cast<int64_t>(blockIdx.x) * kNrBlockRows + w * WR;
    float lo = INFINITY, hi = -INFINITY;
    bool bad = false;
    for (int g = 0; g < WR; g += kNrGroup) {
        float s[kNrGroup];
#pragma unroll
        for (int q = 0; q < kNrGroup; ++q) s[q] = 0.f;
        for (int c = lane; c < Dp; c += 64) {
            float v[kNrGroup];
#pragma unroll
            for (int q = 0; q < kNrGroup; ++q) {
                const int64_t row = r0 + g + q;
                v[q] = row < N ? X[row * Dp + c] : 0.f;
            }
#pragma unroll
            for (int q = 0; q < kNrGroup; ++q) {
                if (r0 + g + q < N) {
                    s[q] = fmaf(v[q], v[q], s[q]);
                    bad |= !(v[q] == rintf(v[q])) || !(fabsf(v[q]) < 1e9f);
                    lo = fminf(lo, v[q]);
                    hi = fmaxf(hi, v[q]);
                }
            }
        }
#pragma unroll
        for (int q = 0; q < kNrGroup; ++q) {
#pragma unroll
            for (int o = 32; o > 0; o >>= 1) s[q] += __shfl_xor(s[q], o);
            if (lane == 0 && r0 + g + q < N) norms[r0 + g + q] = s[q];
        }
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        lo = fminf(lo, __shfl_xor(lo, o));
        hi = fmaxf(hi, __shfl_xor(hi, o));
    }
    const bool any_bad = __ballot(bad) != 0;
    if (lane == 0) {
        const bool any_row = r0 < N;
        red[w][0] = any_bad ? 1 : 0;
        red[w][1] = any_row && !any_bad ? static_cast<int>(lo) : INT_MAX;
        red[w][2] = any_row && !any_bad ? static_cast<int>(hi) : INT_MIN;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        int f = 0, mn = INT_MAX, mx = INT_MIN;
        for (int q = 0; q < 4; ++q) {
            f |= red[q][0];
            mn = min(mn, red[q][1]);
            mx = max(mx, red[q][2]);
        }
        part[3 * blockIdx.x] = f;
        part[3 * blockIdx.x + 1] = mn;
        part[3 * blockIdx.x + 2] = mx;
    }
}

__global__ void __launch_bounds__(1024) int_range_final_kernel(const int* __restrict__ part, int64_t nb,
                                                               int* __restrict__ out)
{
    __shared__ int red[16][3];
    int f = 0, mn = INT_MAX, mx = INT_MIN;
    for (int64_t b = threadIdx.x; b < nb; b += 1024) {
        f |= part[3 * b];
        mn = min(mn, part[3 * b + 1]);
        mx = max(mx, part[3 * b + 2]);
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        f |= __shfl_xor(f, o);
        mn = min(mn, __shfl_xor(mn, o));
        mx = max(mx, __shfl_xor(mx, o));
    }
    const int w = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 0) { red[w][0] = f; red[w][1] = mn; red[w][2] = mx; }
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int q = 1; q < 16; ++q) { f |= red[q][0]; mn = min(mn, red[q][1]); mx = max(mx, red[q][2]); }
        out[0] = f;
        out[1] = mn;
        out[2] = mx;
    }
}

// Exact int8 rows (value - shift, columns >= D zero) and their |x|^2, one
// wave per row, 4 columns per lane.
__global__ void __launch_bounds__(256) quantize_norms_i8_kernel(const float* __restrict__ src, int64_t N, int D,
                                                                int Dp, int shift, int8_t* __restrict__ dst,
                                                                float* __restrict__ norms)
{
    const int64_t row = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (row >= N) return;
    int s = 0;
    for (int c0 = 4 * lane; c0 < Dp; c0 += 256) {
        uint32_t packed = 0;
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const int c = c0 + u;
            const float v = c < D ? rintf(src[row * Dp + c] - static_cast<float>(shift)) : 0.f;
            const int q = static_cast<int>(fminf(fmaxf(v, -128.f), 127.f));
            s += q * q;
            packed |= (static_cast<uint32_t>(q) & 0xffu) << (8 * u);
        }
        *reinterpret_cast<uint32_t*>(dst + row * Dp + c0) = packed;
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) s += __shfl_xor(s, o);
    if (lane == 0) norms[row] = static_cast<float>(s);
}

// quantize_norms_i8_kernel over float4 loads: a block takes kQnBlockRows
// contiguous rows as one flat run of float4s (four loads in flight per
// thread); a row's |x|^2 is summed in LDS (integers, any order).
constexpr int kQnBlockRows = 64;
__global__ void __launch_bounds__(256) quantize_norms_i8_vec_kernel(const float4* __restrict__ src, int64_t N, int D,
                                                                    int Dp, int shift, uint32_t* __restrict__ dst,
                                                                    float* __restrict__ norms)
{
    __shared__ int sn[kQnBlockRows];
    const int tid = threadIdx.x;
    const int64_t r0 = static_cast<int64_t>(blockIdx.x) * kQnBlockRows;
    const int rows = static_cast<int>(N - r0 < kQnBlockRows ? N - r0 : kQnBlockRows);
    if (tid < kQnBlockRows) sn[tid] = 0;
    __syncthreads();
    const int F4 = Dp / 4;
    const int total = rows * F4;
    const int64_t base = r0 * F4;
    const float fs = static_cast<float>(shift);
    for (int e0 = tid; e0 < total; e0 += 256 * 4) {
        float4 v[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const int e = e0 + 256 * u;
            v[u] = e < total ? src[base + e] : make_float4(0.f, 0.f, 0.f, 0.f);
        }
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const int e = e0 + 256 * u;
            if (e < total) {
                const int row = e / F4, c0 = (e - row * F4) * 4;
                const float x[4] = {v[u].x, v[u].y, v[u].z, v[u].w};
                uint32_t packed = 0;
                int sq = 0;
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    const float t = c0 + k < D ? rintf(x[k] - fs) : 0.f;
                    const int q = static_cast<int>(fminf(fmaxf(t, -128.f), 127.f));
                    sq += q * q;
                    packed |= (static_cast<uint32_t>(q) & 0xffu) << (8 * k);
                }
                dst[base + e] = packed;
                atomicAdd(&sn[row], sq);
            }
        }
    }
    __syncthreads();
    if (tid < rows) norms[r0 + tid] = static_cast<float>(sn[tid]);
}

void launch_row_norms_range(const float* X, int64_t N, int Dp, float* norms, int* part, int* out, hipStream_t s)
{
    if (N <= 0) return;
    const int64_t nb = (N + kNrBlockRows - 1) / kNrBlockRows;
    hipLaunchKernelGGL(row_norms_range_kernel, dim3(static_cast<unsigned>(nb)), dim3(256), 0, s, X, N, Dp, norms, part);
    hipLaunchKernelGGL(int_range_final_kernel, dim3(1), dim3(1024), 0, s, part, nb, out);
    GT_HIP(hipGetLastError());
}

void launch_quantize_norms_i8(const float* src, int64_t N, int D, int Dp, int shift, int8_t* dst, float* norms,
                              hipStream_t s)
{
    if (N <= 0) return;
    if (Dp % 4 == 0 && reinterpret_cast<uintptr_t>(src) % 16 == 0 && reinterpret_cast<uintptr_t>(dst) % 4 == 0)
        hipLaunchKernelGGL(quantize_norms_i8_vec_kernel, dim3(static_cast<unsigned>(ceil_div(N, kQnBlockRows))),
                           dim3(256), 0, s, reinterpret_cast<const float4*>(src), N, D, Dp, shift,
                           reinterpret_cast<uint32_t*>(dst), norms);
    else
        hipLaunchKernelGGL(quantize_norms_i8_kernel, dim3(grid_for(N, 4)), dim3(256), 0, s, src, N, D, Dp, shift,
                           dst, norms);
    GT_HIP(hipGetLastError());
}


void launch_quantize_i8(const float* src, int64_t N, int D, int Dp, int shift, int8_t* dst, hipStream_t s)
{
    if (N * Dp <= 0) return;
    hipLaunchKernelGGL(quantize_i8_kernel, dim3(grid_for(N * Dp, 256)), dim3(256), 0, s, src, N, D, Dp, shift, dst);
    GT_HIP(hipGetLastError());
}

void launch_round_to_int(const float* src, int64_t N, int D, int Dp, int shift, float* dst, hipStream_t s)
{
    if (N * Dp <= 0) return;
    hipLaunchKernelGGL(round_to_int_kernel, dim3(grid_for(N * Dp, 256)), dim3(256), 0, s, src, N, D, Dp, shift, dst);
    GT_HIP(hipGetLastError());
}

void launch_row_norms_i8(const int8_t* X, int64_t N, int Dp, float* norms, hipStream_t s)
{
    if (N <= 0) return;
    hipLaunchKernelGGL(row_norms_i8_kernel, dim3(grid_for(N, 4)), dim3(256), 0, s, X, N, Dp, norms);
    GT_HIP(hipGetLastError());
}

void launch_row_norms(const float* X, int64_t N, int Dp, float* norms, hipStream_t s)
{
    if (N <= 0) return;
    hipLaunchKernelGGL(row_norms_kernel, dim3(grid_for(N, 4)), dim3(256), 0, s, X, N, Dp, norms);
    GT_HIP(hipGetLastError());
}

void launch_copy_ranges(const void* tasks, int64_t ntasks, const int32_t* members, int32_t* pool, hipStream_t s)
{
    if (ntasks <= 0) return;
    hipLaunchKernelGGL(copy_ranges_kernel, dim3(static_cast<unsigned>(ntasks)), dim3(256), 0, s,
                       static_cast<const CopyTask*>(tasks), members, pool);
    GT_HIP(hipGetLastError());
}

void launch_negate(float* d, int64_t n, hipStream_t s)
{
    if (n <= 0) return;
    hipLaunchKernelGGL(negate_kernel, dim3(grid_for(n, 256)), dim3(256), 0, s, d, n);
    GT_HIP(hipGetLastError());
}

__global__ void init_flags_kernel(unsigned long long* __restrict__ bad_row, int* __restrict__ err)
{
    if (threadIdx.x == 0) {
        *bad_row = ~0ull;
        *err = 0;
    }
}

void launch_init_flags(unsigned long long* bad_row, int* err, hipStream_t s)
{
    hipLaunchKernelGGL(init_flags_kernel, dim3(1), dim3(64), 0, s, bad_row, err);
    GT_HIP(hipGetLastError());
}

void launch_sanitize(const int32_t* in, int64_t N, int M, uint32_t* out, hipStream_t s)
{
    if (N <= 0) return;
    const bool vec = (reinterpret_cast<uintptr_t>(in) | reinterpret_cast<uintptr_t>(out)) % 16 == 0;
#define GT_SAN_VEC(LL)                                                                                          \
    hipLaunchKernelGGL((sanitize_vec_kernel<LL>), dim3(grid_for(N, 4 * (64 / LL))), dim3(256), 0, s,            \
                       reinterpret_cast<const int4*>(in), N, reinterpret_cast<uint4*>(out))
    if (vec && M == 64) GT_SAN_VEC(16);
    else if (vec && M == 32) GT_SAN_VEC(8);
    else if (vec && M == 128) GT_SAN_VEC(32);
    else if (vec && M == 16) GT_SAN_VEC(4);
    else hipLaunchKernelGGL(sanitize_kernel, dim3(grid_for(N, 4)), dim3(256), 0, s, in, N, M, out);
#undef GT_SAN_VEC
    GT_HIP(hipGetLastError());
}

void launch_cagra_prune(const int32_t* G, int64_t N, int M, int K, uint32_t* out, unsigned long long* bad_row,
                        hipStream_t s, const int32_t* order, bool flat_rows)
{
    GT_REQUIRE(M >= 1 && M <= kPruneMaxM, "prune supports intermediate degree <= 128");
    if (N <= 0) return;
    PruneMap m{};
    m.order = order;
    const dim3 grid(static_cast<unsigned>(8 * ceil_div(ceil_div(N, int64_t(4)), int64_t(8))));
    // buffer loads need byte offsets and the buffer size in 31 bits; larger
    // tables (and flat_rows) take 64-bit addresses
    const bool buf = !flat_rows && N * M * 4 < (int64_t(1) << 31);
    if (M <= 64 && buf)
        hipLaunchKernelGGL((cagra_prune_kernel<1, 0, true>), grid, dim3(256), 0, s, G, N, M, K, out, bad_row, m);
    else if (M <= 64)
        hipLaunchKernelGGL((cagra_prune_kernel<1, 0>), grid, dim3(256), 0, s, G, N, M, K, out, bad_row, m);
    else if (buf)
        hipLaunchKernelGGL((cagra_prune_kernel<2, 0, true>), grid, dim3(256), 0, s, G, N, M, K, out, bad_row, m);
    else
        hipLaunchKernelGGL((cagra_prune_kernel<2, 0>), grid, dim3(256), 0, s, G, N, M, K, out, bad_row, m);
    GT_HIP(hipGetLastError());
}

void launch_cagra_prune_mapped(const int32_t* G, int64_t N, int M, int K, uint32_t* out, unsigned long long* bad_row,
                               const PruneMap& map, int rows_mode, hipStream_t s)
{
    GT_REQUIRE(M >= 1 && M <= kPruneMaxM, "prune supports intermediate degree <= 128");
    GT_REQUIRE(rows_mode == 1 || rows_mode == 2, "bad prune row mode");
    if (map.n <= 0) return;
#define GT_PRUNE_MAP(EE, RR)                                                                                   \
    hipLaunchKernelGGL((cagra_prune_kernel<EE, RR>), dim3(grid_for(map.n, 4)), dim3(256), 0, s, G, N, M, K, out, \
                       bad_row, map)
    if (M <= 64) {
        if (rows_mode == 1) GT_PRUNE_MAP(1, 1);
        else GT_PRUNE_MAP(1, 2);
    } else {
        if (rows_mode == 1) GT_PRUNE_MAP(2, 1);
        else GT_PRUNE_MAP(2, 2);
    }
#undef GT_PRUNE_MAP
    GT_HIP(hipGetLastError());
}

void launch_rev_count(const uint32_t* fwd, int64_t N, int K, uint32_t* deg, uint32_t* slot, int* err, hipStream_t s)
{
    const int64_t E = N * K;
    if (E <= 0) return;
    hipLaunchKernelGGL(rev_count_kernel, dim3(grid_for(E, 256)), dim3(256), 0, s, fwd, E, N, deg, slot, err);
    GT_HIP(hipGetLastError());
}

void launch_exclusive_scan(const uint32_t* in, int64_t n, uint32_t* out, uint32_t* sums, hipStream_t s)
{
    const int64_t nb = (n + kScanBlock - 1) / kScanBlock;
    if (n > 0) hipLaunchKernelGGL(scan_block_kernel, dim3(static_cast<unsigned>(nb)), dim3(256), 0, s, in, n, out, sums);
    hipLaunchKernelGGL(scan_sums_kernel, dim3(1), dim3(256), 0, s, sums, nb, out + n);
    if (n > 0) hipLaunchKernelGGL(scan_add_kernel, dim3(grid_for(n, 256)), dim3(256), 0, s, out, n, sums);
    GT_HIP(hipGetLastError());
}

void launch_rev_scatter(const uint32_t* fwd, int64_t N, int K, const uint32_t* off, const uint32_t* slot,
                        unsigned long long* keys, hipStream_t s)
{
    const int64_t E = N * K;
    if (E <= 0) return;
    hipLaunchKernelGGL(rev_scatter_kernel, dim3(grid_for(E, 256)), dim3(256), 0, s, fwd, E, N, K, off, slot, keys);
    GT_HIP(hipGetLastError());
}

// Bin shift of the binned path, or -1 when N is beyond its limits.
int rev_bin_shift(int64_t N)
{
    int sh = 5;
    while (sh < kRevMaxBinShift && ceil_div(N, int64_t(1) << sh) > 4096) ++sh;
    return ceil_div(N, int64_t(1) << sh) <= kRevMaxBins ? sh : -1;
}

int rev_bin_blocks(int64_t E) { return static_cast<int>(std::max<int64_t>(1, std::min<int64_t>(512, ceil_div(E, 8192)))); }

void launch_rev_binned(const uint32_t* fwd, int64_t N, int K, uint32_t* hist, uint32_t* offs, uint32_t* sums,
                       unsigned long long* part, unsigned long long* grouped, uint32_t* out, int* err, hipStream_t s)
{
    GT_REQUIRE(K >= 1 && K <= kRevMaxK, "reverse merge supports output degree <= 64");
    const int shift = rev_bin_shift(N);
    GT_REQUIRE(shift >= 0, "binned reverse merge: too many rows");
    const int64_t E = N * K;
    if (E <= 0) return;
    const int nbins = static_cast<int>(ceil_div(N, int64_t(1) << shift));
    const int nblk = rev_bin_blocks(E);
    const int64_t chunk = ceil_div(E, nblk);
    // LDS of (1)-(3) sized to the bins in use, so that several blocks share a CU
    const size_t lds_bins = static_cast<size_t>(nbins) * sizeof(uint32_t);
    hipLaunchKernelGGL(rev_bin_count_kernel, dim3(nblk), dim3(kRevBinThreads), lds_bins, s, fwd, E, N, chunk, shift,
                       nbins, hist, err);
    launch_exclusive_scan(hist, static_cast<int64_t>(nbins) * nblk, offs, sums, s);
    hipLaunchKernelGGL(rev_bin_scatter_kernel, dim3(nblk), dim3(kRevBinThreads), lds_bins, s, fwd, E, N, K, chunk,
                       shift, nbins, offs, part);
    const size_t lds = (2 * (size_t(1) << shift) + 1) * sizeof(uint32_t);
    hipLaunchKernelGGL(rev_bin_merge_kernel, dim3(nbins), dim3(kRevBinThreads), lds, s, fwd, N, K, shift, nblk, offs,
                       part, grouped, out);
    GT_HIP(hipGetLastError());
}

void launch_rev_merge(const uint32_t* fwd, int64_t N, int K, const uint32_t* off, const unsigned long long* keys,
                      uint32_t* out, hipStream_t s)
{
    GT_REQUIRE(K >= 1 && K <= kRevMaxK, "reverse merge supports output degree <= 64");
    if (N <= 0) return;
    hipLaunchKernelGGL(rev_merge_kernel, dim3(grid_for(N, 4)), dim3(256), 0, s, fwd, N, K, off, keys, out);
    GT_HIP(hipGetLastError());
}

void launch_merge_rounds(const int32_t* ri, const float* rd, const int32_t* ni, const float* nd, int64_t N, int M,
                         int32_t* oi, float* od, hipStream_t s)
{
    GT_REQUIRE(M >= 1 && M <= kMergeMaxM, "merge supports list length <= 128");
    if (N <= 0) return;
    const int64_t g = std::min<int64_t>(grid_for(N, 4), kMergeBlocks);
    hipLaunchKernelGGL(merge_rounds_kernel, dim3(static_cast<unsigned>(g)), dim3(256), 0, s, ri, rd, ni, nd, N, M,
                       oi, od);
    GT_HIP(hipGetLastError());
}

void launch_invert_perm(const uint32_t* inv, int64_t N, uint32_t* perm, uint32_t* hits, int* err, hipStream_t s)
{
    if (N <= 0) return;
    hipLaunchKernelGGL(invert_perm_kernel, dim3(grid_for(N, 256)), dim3(256), 0, s, inv, N, perm, hits, err);
    hipLaunchKernelGGL(check_hits_kernel, dim3(grid_for(N, 256)), dim3(256), 0, s, hits, N, err);
    GT_HIP(hipGetLastError());
}

void launch_permute_rows(const void* in, const uint32_t* inv, int64_t N, int64_t row_bytes, void* out, hipStream_t s)
{
    if (N <= 0 || row_bytes <= 0) return;
    const dim3 grid(grid_for(N, 4));
    const uintptr_t al = reinterpret_cast<uintptr_t>(in) | reinterpret_cast<uintptr_t>(out);
    if (row_bytes % 16 == 0 && al % 16 == 0)
        hipLaunchKernelGGL(permute_rows_kernel<uint4>, grid, dim3(256), 0, s, static_cast<const uint4*>(in), inv, N,
                           row_bytes / 16, static_cast<uint4*>(out));
    else if (row_bytes % 4 == 0 && al % 4 == 0)
        hipLaunchKernelGGL(permute_rows_kernel<uint32_t>, grid, dim3(256), 0, s, static_cast<const uint32_t*>(in),
                           inv, N, row_bytes / 4, static_cast<uint32_t*>(out));
    else
        hipLaunchKernelGGL(permute_rows_kernel<uint8_t>, grid, dim3(256), 0, s, static_cast<const uint8_t*>(in), inv,
                           N, row_bytes, static_cast<uint8_t*>(out));
    GT_HIP(hipGetLastError());
}

void launch_remap_table(const int32_t* ids, const uint32_t* inv, const uint32_t* perm, int64_t N, int M, int32_t* out,
                        hipStream_t s)
{
    if (N * M <= 0) return;
    hipLaunchKernelGGL(remap_table_kernel, dim3(grid_for(N * M, 256)), dim3(256), 0, s, ids, inv, perm, N, M, out);
    GT_HIP(hipGetLastError());
}

void launch_translate(const uint32_t* g, const uint32_t* inv, int64_t N, int K, uint32_t* out, uint32_t* hits,
                      int* err, hipStream_t s)
{
    if (N * K <= 0) return;
    hipLaunchKernelGGL(translate_kernel, dim3(grid_for(N * K, 256)), dim3(256), 0, s, g, inv, N, K, out, hits, err);
    hipLaunchKernelGGL(check_hits_kernel, dim3(grid_for(N, 256)), dim3(256), 0, s, hits, N, err);
    GT_HIP(hipGetLastError());
}

}  // namespace gtann
