// gtann_common.hpp -- shared definitions of the gfx950 graph-build library.
#pragma once

#include <hip/hip_runtime.h>

#include "../../include/gtann.h"

#include <cstdint>
#include <stdexcept>
#include <string>

namespace gtann {

struct Error : std::runtime_error {
    int code;
    Error(int c, const std::string& m) : std::runtime_error(m), code(c) {}
};

#define GT_HIP(call)                                                                         \
    do {                                                                                     \
        hipError_t e_ = (call);                                                              \
        if (e_ != hipSuccess)                                                                \
            throw ::gtann::Error(e_ == hipErrorOutOfMemory ? GT_ENOMEM                        \
                                                           : GT_EDEVICE,                     \
                                 std::string(#call) + ": " + hipGetErrorString(e_) + " at " + \
                                     __FILE__ + ":" + std::to_string(__LINE__));             \
    } while (0)

#define GT_REQUIRE(cond, msg)                                                  \
    do {                                                                       \
        if (!(cond)) throw ::gtann::Error(GT_EINVAL, std::string(msg));          \
    } while (0)

// One unit of work of the fused distance/top-M kernel: a tile of up to
// kQueriesPerBlock query rows (a contiguous slice of the query list) scanned
// against a contiguous slice of the pool list.
struct WorkItem {
    int64_t q_begin;    // first index into the query list
    int64_t p_begin;    // first index into the pool list
    int64_t out_base;   // >= 0: output row of query q_begin (partial lists); < 0: row = query id
    int32_t q_count;
    int32_t p_count;
    int32_t p_rot = 0;  // the scan visits pool positions p_rot, p_rot+1, ... (mod p_count)
};

constexpr int kQueriesPerWave = 32;
constexpr int kWaves = 4;
constexpr int kQueriesPerBlock = kQueriesPerWave * kWaves;   // 128
constexpr int kPoolTile = 32;

// Arguments of the fused distance + top-M kernel.
struct KnnArgs {
    const float* Xq;        // query vectors, row stride Dp (zero padded)
    const float* Xp;        // pool vectors, row stride Dp
    const float* nq;        // |x|^2 of query rows (indexed by query row id)
    const float* np;        // |x|^2 of pool rows (indexed by pool row id)
    const int32_t* q_rows;  // query list (row ids into Xq); nullptr = identity
    const int32_t* p_rows;  // pool list (row ids into Xp); nullptr = identity
    const WorkItem* items;
    int32_t n_items;
    int32_t Dp;
    int32_t M;              // list length
    int32_t metric;         // 0 = L2, 1 = inner product (key = -<x,y>)
    int32_t exclude_self;   // drop pool entries whose row id equals the query row id
    int32_t out_pos;        // write pool-list positions instead of row ids
    const float* seed_d;    // optional per-query cap on kept keys: seed_d[orow * seed_ld + seed_ld - 1], orow = output row
    int32_t seed_ld;
    int32_t* out_ids;       // (rows, M)
    float* out_d;           // (rows, M)
    // int8 operands (integer-typed inputs): when set, the int8 kernel runs
    // on these rows (stride Dp bytes) and nq/np are their |x|^2
    const int8_t* Xq8;
    const int8_t* Xp8;
    // collect launches (knn_collect.hip): the keys of a query at or below its
    // threshold go to cand[row * kCollectCap ...), their number to cand_cnt[row]
    uint64_t* cand;
    int32_t* cand_cnt;
    unsigned long long* stats;   // optional: [0] keys collected, [1] compactions, [2] tiles past the
                                 // pre-filter, [3] tiles filtered (per wave)
    // exact chunk pruning of the int8 collect kernel (L2): every pool starts
    // at a multiple of kChunkRows in the pool list, and chunk g (pool-list
    // rows [kChunkRows g, kChunkRows g + kChunkRows)) has the rounded centre
    // ch8[g * Dp ..] (int8), its |c|^2 chn[g] and chr[g] >= the largest
    // |p - c| of its rows; null = every stage is scanned
    const int8_t* ch8;
    const float* chn;
    const float* chr;
    unsigned long long* pairs_done;   // optional: += (query, pool row) pairs the MFMAs computed
    // collect launches: when set, the new lists are merged into the running
    // table (run_ids, run_d) (rows, M) in place instead of written to
    // (out_ids, out_d), which then hold only the rows the selection took (fp32)
    int32_t* run_ids;
    float* run_d;
    int32_t* hl_rows;      // (rows): int8 merge: the rows left to the selection
    uint32_t* hl_count;    // their number
    int32_t window_tiles;  // collect launches, unseeded: tiles of the threshold window (0: 16)
};

constexpr int kChunkRows = 64;       // pool rows per pruning chunk (= one collect stage)
constexpr int kMaxChunkWords = 24;   // pools of up to 24 * 32 chunks (49,152 rows) are pruned

constexpr int kCollectCap = 256;   // candidate slots per query of a collect launch

// Arguments of the graph search kernel (one wave per query).
struct SearchArgs {
    const float* X;           // base rows, stride Dp, zero padded
    int64_t N;
    int32_t D;
    int32_t Dp;
    const uint32_t* graph;    // (N, deg); entries >= N are skipped
    int32_t deg;
    const float* Q;           // query rows, stride Dp
    const int32_t* entries;   // (nq, n_entry), processed in order; < 0 or >= N skipped
    int32_t n_entry;          // <= 64
    const int32_t* q_list;    // queries to run; nullptr = 0 .. n_run-1
    int64_t n_run;
    int32_t topk;
    int32_t ef;
    int32_t metric;           // 0 = L2, 1 = inner product (key = -<q,x>)
    int32_t H;                // LDS visited table slots (power of two >= 512); 0 = bitmap mode
    int32_t CC;               // candidate capacity (multiple of 64)
    int32_t efr;              // ef rounded up to a multiple of 64
    uint32_t* bitmap;         // bitmap mode: gridDim.x slots of bm_words words, zero on entry
    int64_t bm_words;
    int32_t* out_ids;         // (nq, topk)
    float* out_d;             // (nq, topk)
    int32_t* status;          // (nq): 0 done, 1 visited table full, 2 candidate capacity exceeded
    int32_t* expansions;      // (nq)
    int32_t* visits;          // (nq): points whose distance was computed
};

inline int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }

// Where the rows of a chunked prune live (cagra_prune_kernel, ROWS 1 and 2).
struct PruneMap {
    const int32_t* order;     // ROWS 0: processing order (a permutation of the rows) or null
    int64_t a0, n;            // rows pruned: a0 .. a0 + n - 1, output rows 0 .. n - 1
    const int32_t* cidx;      // ROWS 1: compact row of every id the chunk reads
    const uint32_t* off;      // ROWS 2: n_buckets + 1 row starts, by processing position
    const int32_t* win;       // ROWS 2: (n_buckets, W) window positions
    const int32_t* win_len;   // ROWS 2: (n_buckets)
    const int64_t* cbase;     // ROWS 2: compact row of off[q], -1 = position q not loaded
    int32_t n_buckets;
    int32_t W;
};

// Launch plan of the two-kernel reverse merge (revmerge_kernels.hip).
struct RvPlan {
    int cshift;     // rows per destination bin = 2^cshift
    int nbins;
    int nblk;       // key blocks seen by the merge, each owning spb consecutive source rows
    int64_t spb;
    int kbits, sbits, nbits;   // bits of rank, source within block, source id
    int rp;         // rows per merge pass (= merge block size)
    int cap;        // keys grouped in LDS per pass
    int cap_big;    // the same for the deferred (large) bins
    int bsh = 31;   // bins per superbin = 2^bsh (two levels; 31: one level)
    uint32_t region = 0;   // words per key block in the merge's key array
    // two levels: the scatter first groups by superbin (2^sshift rows, G of
    // them) in nblk1 blocks of spb1 source rows (sbits1 bits), then regroups
    // each superbin's runs of F consecutive level-one blocks by bin
    bool two = false;
    int sshift = 0, G = 0, F = 0, nblk1 = 0, sbits1 = 0;
    int64_t spb1 = 0;
};

// Device buffers of the two-kernel reverse merge: the merge's key blocks and
// their run offsets (block-major, then bin-major), and with two levels the
// level-one keys and offsets.  Sizes in elements (rv_sizes).
struct RvBufs {
    uint32_t* part = nullptr;
    uint16_t* meta_blk = nullptr;
    uint16_t* meta = nullptr;
    uint32_t* part1 = nullptr;
    uint16_t* meta1 = nullptr;
};
struct RvSizes {
    size_t part = 0, meta = 0, part1 = 0, meta1 = 0;
};

// Orders LDS traffic of one wave across its lanes (no s_barrier needed
// inside a wave).
__device__ __forceinline__ void wave_sync()
{
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Order-preserving packing of (key, id): unsigned comparison of the 64-bit
// words is the (key, id) order, ids compared as unsigned (-1 sorts last).
// ~0 is the sentinel (after every real entry).
constexpr uint64_t kNoKey = ~0ull;
__device__ __forceinline__ uint32_t f2o(float f)
{
    const uint32_t u = __float_as_uint(f);
    return u ^ (static_cast<uint32_t>(static_cast<int32_t>(u) >> 31) | 0x80000000u);
}
__device__ __forceinline__ float o2f(uint32_t k)
{
    return __uint_as_float(k ^ ((k & 0x80000000u) ? 0x80000000u : 0xFFFFFFFFu));
}
__device__ __forceinline__ uint64_t pack_key(float d, int32_t id)
{
    return (static_cast<uint64_t>(f2o(d)) << 32) | static_cast<uint32_t>(id);
}
// (distance, id) order of the cross-round merge: distances as floats, ties
// by id; lower_bound_g = the number of entries of a list ascending in that
// order that precede (kd, ki)
__device__ __forceinline__ bool key_less_g(float da, int32_t ia, float db, int32_t ib)
{
    return da < db || (da == db && ia < ib);
}
__device__ __forceinline__ int lower_bound_g(const float* ad, const int32_t* ai, int n, float kd, int32_t ki)
{
    int lo = 0, hi = n;
    while (lo < hi) {
        const int mid = (lo + hi) >> 1;
        if (key_less_g(ad[mid], ai[mid], kd, ki)) lo = mid + 1;
        else hi = mid;
    }
    return lo;
}
__device__ __forceinline__ uint64_t shfl_xor_u64(uint64_t v, int m)
{
    const uint32_t lo = static_cast<uint32_t>(__shfl_xor(static_cast<int>(v), m));
    const uint32_t hi = static_cast<uint32_t>(__shfl_xor(static_cast<int>(v >> 32), m));
    return (static_cast<uint64_t>(hi) << 32) | lo;
}

}  // namespace gtann
