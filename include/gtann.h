/*
 * gtann.h -- C ABI of the MI355X (gfx950) bucketed CAGRA-style graph build.
 *
 * Every entry point takes plain pointers and sizes.  Pointers may refer to
 * host memory or to device memory of the context's GPU (detected per
 * pointer): host buffers are staged through the device and the call
 * returns after the results are back; device buffers are used in place.
 * Calls are synchronous on the context's stream.  One context per host
 * thread; distinct contexts may be used concurrently.
 *
 * Ordering of device buffers: the context's stream is a blocking stream, so
 * a call's reads come after all work queued before the call on the device's
 * legacy null (default) stream -- the stream PyTorch and most HIP callers
 * use by default.  A caller that produces an input on another non-blocking
 * stream must synchronise that stream (or the device) before the call.
 * Every call has finished writing its outputs when it returns.
 *
 * Return value: GT_OK (0) or a negative error code; gt_last_error() gives
 * the message.  No C++ exception crosses this boundary.
 *
 * Conventions: kNN rows are ascending by (distance, id), padding is
 * (-1, +inf).  L2 distances are squared.  For GT_METRIC_IP rows are
 * descending by inner product and the distance slots hold the inner
 * product (padding -inf).
 */
#ifndef GTANN_H
#define GTANN_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct gt_ctx gt_ctx;

enum { GT_OK = 0, GT_EINVAL = -1, GT_ENOMEM = -2, GT_EDEVICE = -3, GT_EFEWCAND = -4 };
enum { GT_DTYPE_F32 = 0, GT_DTYPE_U8 = 1, GT_DTYPE_I8 = 2 };
enum { GT_METRIC_L2 = 0, GT_METRIC_IP = 1 };
enum { GT_SEED_AUTO = 0, GT_SEED_KMEANS_PAR = 1, GT_SEED_UNIFORM = 2 };

/* Context owning a device, a stream and reusable workspaces.
 * Replaces the GpuResidentKnn constructor/destructor
 * (src/bucket.cu:5216-5241, :5650) and the cuVS raft::resources handle. */
int gt_create(int device, gt_ctx** out);
void gt_destroy(gt_ctx* ctx);
/* The message of the context's last error; with ctx NULL, that of this
 * thread's last failed host-only call (gt_bucket_order, gt_bucket_reorder,
 * which accept a NULL context for host buffers), else "null context". */
const char* gt_last_error(const gt_ctx* ctx);
const char* gt_version(void);

/* Exact kNN of the query rows `queries[0..nq)` (all N rows when queries is
 * NULL, then nq must be N) against all N rows, self excluded.
 * ids/dists: nq x k.  Replaces bd/build_knn.py:98-149 (build_exact_knn). */
int gt_knn_exact(gt_ctx* ctx, const void* X, int64_t N, int32_t D, int dtype, int metric,
                 const int64_t* queries, int64_t nq, int32_t k, int32_t* ids, float* dists);

/* Exact top-2 nearest of nC centroid rows C (nC x D, same dtype as X) for
 * each of the N rows of X; ties by lower centroid index.
 * Replaces step4_top2_kernel + its cuBLAS GEMM (src/bucket.cu:1230, :2061-2177). */
int gt_assign_top2(gt_ctx* ctx, const void* X, int64_t N, int32_t D, int dtype, int metric,
                   const void* C, int64_t nC, uint32_t* top2, float* d2);

/* One round of bucketed kNN.  Bucket b owns members[offsets[b]..offsets[b+1])
 * (every point in exactly one bucket); its pool is its own members followed
 * by the members of probe[b*P .. b*P+P) (ids >= nB skipped).  Each point gets
 * the M nearest pool points other than itself.  merge = 0: ids/dists (N x M)
 * are outputs.  merge = 1: ids/dists hold the running table on input (rows
 * ascending by (distance, id), padding (-1, +inf) last, as this call writes
 * them) and the merged table (top-M of both, duplicates once) on output; a
 * row with no new pool point within its running M-th distance keeps its
 * running list as it is.  On integer rows the running distances must be
 * the exact ones this library computes (a table from an earlier call or
 * from gt_knn_exact): the merge drops a new key whose id the running row
 * holds before taking the top M, which equals the merge of the top M only
 * when a pair's distance is the same in both.
 * Replaces GpuResidentKnn::run_round (src/bucket.cu:5310-5546). */
int gt_knn_bucketed(gt_ctx* ctx, const void* X, int64_t N, int32_t D, int dtype, int metric,
                    const int64_t* offsets, const int32_t* members, int64_t nB,
                    const int32_t* probe, int32_t P, int32_t M,
                    int32_t* ids, float* dists, int merge);

/* Cross-round merge of two N x M tables into out (may alias run).
 * Replaces resident_merge_kernel (src/bucket.cu:5021-5130). */
int gt_merge_rounds(gt_ctx* ctx, const int32_t* run_ids, const float* run_d,
                    const int32_t* new_ids, const float* new_d, int64_t N, int32_t M,
                    int32_t* out_ids, float* out_d);

/* `passes` passes of 2-hop local-join refinement of an N x M table in place
 * (S = neighbours sampled per hop, S*S <= 1024).
 * Replaces GpuResidentKnn::refine_local_join / a1_pull_join_kernel
 * (src/bucket.cu:5591-5648, :4754-4850). */
int gt_refine_2hop(gt_ctx* ctx, const void* X, int64_t N, int32_t D, int dtype, int metric,
                   int32_t M, int32_t S, int32_t passes, int32_t* ids, float* dists);

/* -1 / out-of-range / self entries -> first valid entry of the row, else
 * (i+1) % N.  Replaces sanitize_to_uint32_inplace (src/optimize.cu:89-134). */
int gt_sanitize(gt_ctx* ctx, const int32_t* knn, int64_t N, int32_t M, uint32_t* out);

/* CAGRA rank-based detour-count prune of rows already in rank order
 * (entries >= 2^31 as int32 are padding).  GT_EFEWCAND if a row has fewer
 * than K valid candidates.  Replaces prune_windowed_gpu::run
 * (src/prune_windowed_gpu.hpp:7-39, src/prune_windowed_gpu.cu:422-498) with a
 * full window, and the prune half of cuVS helpers::optimize
 * (src/optimize.cu:396). */
int gt_cagra_prune(gt_ctx* ctx, const uint32_t* knn, int64_t N, int32_t M, int32_t K, uint32_t* out);

/* Reverse-edge merge of a forward graph (N x K, K <= 64) with K/2
 * protected slots.  Replaces optimize_chunked -m E Phase 1+2
 * (src/optimize_chunked.cu:372-407, :1421-1471). */
int gt_reverse_merge(gt_ctx* ctx, const uint32_t* fwd, int64_t N, int32_t K, uint32_t* out);

/* Occlusion prune of bd/prune.py:8-83 (prune_graph), L2: per point the valid
 * candidates of nb (N x M; -1, out-of-range and self dropped) in order of
 * distance to the point (ties by column); a candidate is dropped when an
 * earlier kept one is strictly closer to it than the point is.  out (N x M)
 * holds the kept ids left-aligned, at most max_degree of them (<= 0: no
 * cap), then -1.  M <= 128.  Replaces prune.prune_graph (bd/prune.py:8-19). */
int gt_prune_occlusion(gt_ctx* ctx, const void* X, int64_t N, int32_t D, int dtype, const int32_t* nb, int32_t M,
                       int32_t max_degree, int32_t* out);

/* Reverse-edge insertion of bd/build_bucket.py:473-543 on an N x M table
 * (rows ascending), in place: every edge a -> b with distance d strictly below
 * the largest distance of b's row is offered to b; sources already in b's
 * row are dropped; a row that receives an offer becomes the M smallest of
 * (row, offers) by (distance, id).  M <= 128.
 * Replaces _apply_reverse_edges (bd/build_bucket.py:473). */
int gt_reverse_insert(gt_ctx* ctx, int32_t* ids, float* dists, int64_t N, int32_t M);

/* Reverse merge of a host forward graph (N x K, K <= 64) into host rows out,
 * out of core: the forward rows stream through the device in batches that
 * route every edge to its destination chunk, then one destination chunk at a
 * time is merged, each within device_budget_bytes of device memory (<= 0:
 * one chunk); a chunk whose rows receive more edges than its share (hub
 * rows) is merged in row ranges that fit, and a single row with more
 * in-edges than a chunk's share alone, over the budget by its excess.  Same
 * rows as gt_reverse_merge.  Replaces run_method_E with
 * several chunks (src/optimize_chunked.cu:1548-2057; optimize_chunked -m E
 * --gpu-budget-mb). */
int gt_reverse_merge_chunked(gt_ctx* ctx, const uint32_t* fwd, int64_t N, int32_t K, int64_t device_budget_bytes,
                             uint32_t* out);

/* Windowed CAGRA prune (src/prune_windowed_gpu.cu:529-915, run_chunked;
 * src/prune_windowed_core.hpp:177-263) of host candidate rows cand (N x M,
 * rank order, -1 = padding) in the bucket-contiguous id space: processing
 * position q owns ids [offsets[q], offsets[q+1]) (offsets: n_buckets + 1,
 * offsets[0] = 0, offsets[n_buckets] = N).  A row at position p counts a
 * detour through its neighbour d only when d's position is one of win[p*W ..
 * p*W + win_len[p]) (the reference puts p itself and its centroid-kNN or pool
 * buckets there); a neighbour outside the window contributes nothing (with
 * every position in every window this is gt_cagra_prune).  Then the first K
 * by (count, rank).  Positions go in chunks whose window union fits
 * device_budget_bytes (<= 0: no limit); the rows do not depend on it.  out:
 * host N x K.  GT_EFEWCAND if a row has fewer than K valid candidates. */
int gt_prune_windowed(gt_ctx* ctx, const int32_t* cand, int64_t N, int32_t M, const uint32_t* offsets,
                      int32_t n_buckets, const int32_t* win, const int32_t* win_len, int32_t W, int32_t K,
                      int64_t device_budget_bytes, uint32_t* out);

/* prune then reverse merge.  Replaces cuvs::neighbors::cagra::helpers::optimize
 * (src/optimize.cu:395-397, src/bucket.cu:8470). */
int gt_optimize(gt_ctx* ctx, const uint32_t* knn, int64_t N, int32_t M, int32_t K, uint32_t* out);

/* gt_optimize without any allocation.  No counterpart in the reference: for
 * callers that cannot allocate device memory (tight serving loops, harnesses
 * that forbid hipMalloc).  It is not capturable into a HIP graph: like every
 * call here it runs on the context's stream and synchronises it (the row
 * check reads its error flags back).  knn (N x M) and out
 * (N x K) must be device memory of the context's GPU (GT_EINVAL otherwise).
 * The forward graph, the error flags and the reverse merge's bins and keys
 * live in one fixed device array per GPU (GT_NOALLOC_SCRATCH_BYTES, held by
 * every GPU the library runs on until the process ends), which limits the
 * call to N * K <= GT_NOALLOC_MAX_EDGES (GT_EINVAL beyond).  Every call on a
 * GPU shares that GPU's array: calls that overlap on one GPU (other threads,
 * other contexts) race and must be serialised by the caller.  Same results
 * as gt_optimize, bit for bit. */
#define GT_NOALLOC_MAX_EDGES (1 << 20)
#define GT_NOALLOC_SCRATCH_BYTES (25u << 20)
int gt_optimize_noalloc(gt_ctx* ctx, const uint32_t* knn, int64_t N, int32_t M, int32_t K, uint32_t* out);

/* out[inv[i]][k] = inv[g[i][k]]; GT_EINVAL unless inv is a permutation.
 * Replaces translate_ids::translate_graph_to_original_order
 * (src/translate_graph_ids.hpp:75). */
int gt_translate(gt_ctx* ctx, const uint32_t* g, const uint32_t* inv, int64_t N, int32_t K, uint32_t* out);

/* Defaults (gt_build_params_default): 2 rounds, 3 Lloyd iterations on a
 * training subset, nprobe 1, balance 0.8, M 64, K 32, N/4000 buckets, seed 42.
 * The reference's own settings are rounds 3, kmeans_iters 0 (data points as
 * centroids), nprobe -1 (sk/scripts/params.sh:12, dataset_env.py:56). */
typedef struct gt_build_params {
    int32_t metric;         /* GT_METRIC_L2 / GT_METRIC_IP */
    int32_t n_buckets;      /* buckets per round (--centroid-ratio * N); 0 = N / 4000 */
    int32_t nprobe;         /* probe buckets per bucket (--nprobe); -1 = ceil(20000 / avg bucket) */
    int32_t M;              /* intermediate degree (--neighbors-m) */
    int32_t K;              /* output degree (--fused-optimize-degree) */
    int32_t rounds;         /* rounds with fresh buckets (-t) */
    int32_t refine_passes;  /* 2-hop refinement passes (BUCKET2_A1_PASSES) */
    int32_t refine_sample;  /* S of the refinement (BUCKET2_A1_SAMPLE) */
    int32_t kmeans_iters;   /* Lloyd iterations on a training subset (0 = sampled data points) */
    float balance;          /* two-choice factor: 2nd bucket if size2 < balance*size1 (<= 0 off) */
    uint64_t seed;          /* --seed; round r uses seed + r */
    int32_t reverse_edges;  /* 1: each round's full table gets gt_reverse_insert before the
                               cross-round merge (bd/build_bucket.py:628); 0: rounds seeded */
    int32_t int_exact;      /* 1 (default): float rows whose values are all integers in [-128, 127]
                               or [0, 255] (D <= 256) run the point kNN on the int8 matrix cores;
                               every distance is an exact integer in both kernels, so the table and
                               graph are the fp32 kernel's, bit for bit.  0: always fp32 */
    int32_t device_budget_mb; /* bucket2's --gpu-limit: 0 (default) = the tables live on the device.
                               > 0 and the resident tables exceed it: out of core -- the running
                               N x M table and the graphs stay in host memory and move through this
                               many MiB of device memory chunk by chunk (buckets for the kNN rounds,
                               rows plus their neighbours' rows for the prune, destination rows for
                               the reverse merge); same table and graph.  The dataset stays on the
                               device and is not counted.  Excludes refine_passes and reverse_edges.
                               Replaces ChunkedKnnAccumulator (src/bucket.cu:5670-6369) */
    int32_t seeding;        /* where the centroids start: GT_SEED_AUTO (default) = KMeans|| with
                               kmeans_iters 0 (the reference's Step 2,
                               src/bucket.cu:2833-3168), a uniform sample of rows
                               before Lloyd iterations; GT_SEED_KMEANS_PAR / GT_SEED_UNIFORM force one */
    float kmeans_train_fraction; /* KMeans|| trains on each row with this probability
                               (--kmeans-train-fraction; all rows when fewer than 4 x buckets are
                               kept); <= 0 (default): min(0.1, 1e7 / N), sk/scripts/dataset_env.py:57 */
} gt_build_params;

typedef struct gt_build_stats {
    double t_total;         /* wall seconds of the whole call */
    double t_prepare;       /* upload / convert / norms */
    double t_bucketing;     /* centroids, probe table, top-2, balance, pools */
    double t_knn;           /* fused kNN kernels (device time) */
    double t_merge;         /* cross-round merges (device time) */
    double t_refine;        /* refinement (device time) */
    double t_prune;         /* sanitize + prune (device time) */
    double t_revmerge;      /* reverse-edge merge (device time) */
    double t_download;      /* results to host */
    double knn_flops;       /* algorithmic flops of the distance contraction (2*D per pair) */
    double knn_pairs;       /* (query, pool) pairs scanned */
    int64_t max_pool;
    int64_t max_bucket;
    int64_t knn_launches;   /* fused kNN launches of the rounds (knn_flops / t_knn cover these) */
    int64_t knn_int8;       /* 1: the rounds ran on the int8 matrix cores (integer-typed rows, or
                               integer-valued float rows with int_exact), 0: fp32 */
    int64_t ooc_chunks;     /* device chunks of an out-of-core build (0: resident) */
    double knn_pairs_computed; /* pairs the exact distance kernels computed: knn_pairs less the pool
                               chunks the exact pruning skipped and the pool rows the fp16 screen
                               dropped (the screen itself computes every pair) */
} gt_build_stats;

void gt_build_params_default(gt_build_params* p);

/* The whole bucketed build: `rounds` rounds of (centroids -> probe table ->
 * top-2 assignment with two-choice balance -> pooled kNN -> merge), optional
 * refinement, sanitize, CAGRA prune, reverse merge.  knn_ids/knn_dists
 * (N x M, optional, NULL to skip) receive the pre-prune table, graph
 * (N x K, NULL = stop after the table) the final graph.  Replaces bucket2's GPU-resident path
 * (src/bucket.cu:8729-9842 with --fused-optimize-degree). */
int gt_build_graph(gt_ctx* ctx, const void* X, int64_t N, int32_t D, int dtype,
                   const gt_build_params* params, int32_t* knn_ids, float* knn_dists,
                   uint32_t* graph, gt_build_stats* stats);

/* Optional outputs of gt_build_graph_ex about round 1, from which bucket2's
 * reorder artifacts are made, and about the last round, from which its
 * Step-5 files are (src/bucket.cu:9552-9568).  C = the bucket count
 * (params->n_buckets, or N / 4000 when 0, clamped to [1, N]).  Host or
 * device memory. */
typedef struct gt_build_extras {
    int32_t* round1_bucket;   /* N, or NULL: round-1 bucket of every point */
    uint32_t* centroid_knn;   /* C x centroid_knn_k, or NULL: exact self-kNN of the round-1
                                 centroids (self excluded, ascending distance), as
                                 centroid_self_knn_bf (src/bucket.cu:3241, 8976-8986) */
    int32_t centroid_knn_k;   /* <= min(C - 1, 128) */
    int32_t reserved_;
    int32_t* last_bucket;     /* N, or NULL: last-round bucket of every point (bucket_data.bin) */
    int64_t* last_centroids;  /* C, or NULL: the data point each last-round centroid is (KMeans||
                                 seeds) or was seeded from before its Lloyd iterations
                                 (centroid_global_indices.bin) */
} gt_build_extras;

/* gt_build_graph plus the round-1 extras (NULL = none). */
int gt_build_graph_ex(gt_ctx* ctx, const void* X, int64_t N, int32_t D, int dtype,
                      const gt_build_params* params, int32_t* knn_ids, float* knn_dists,
                      uint32_t* graph, gt_build_stats* stats, const gt_build_extras* extras);

/* DiskJoin bucket processing order over the flat (B x K) bucket graph
 * (entries equal to the row or >= B are dropped): start at the bucket of
 * largest out-degree (ties: smallest id), then repeatedly place the
 * unplaced bucket, among those sharing a neighbour with the last `window`
 * placed ones, of largest summed neighbour overlap with them (ties: larger
 * id), else the smallest unplaced id.  Host-side.  Replaces
 * bucket_order::compute_bucket_processing_order(adjacency_from_flat_graph(...))
 * (src/bucket_order.hpp:161-238, 247-262). */
int gt_bucket_order(gt_ctx* ctx, const uint32_t* graph, int64_t B, int32_t K, int32_t window, int32_t* order);
/* (ctx may be NULL for host buffers, here and in gt_bucket_reorder.) */

/* New-id layout of round-1 buckets in processing order: inverse_perm (N,
 * new id -> old id: each bucket's points in increasing old id, buckets in
 * `order`), bucket_offsets (n_buckets + 1, by processing position) and, for
 * n_cids given old ids (e.g. centroid rows), their new ids (or NULL).
 * Every point must have a bucket in [0, n_buckets).  Host-side.  Replaces
 * compute_bucket_reorder (src/bucket.cu:8363-8412). */
int gt_bucket_reorder(gt_ctx* ctx, const int32_t* assignment, int64_t N, int64_t n_buckets, const int32_t* order,
                      const int64_t* cids, int64_t n_cids, uint32_t* inverse_perm, uint32_t* bucket_offsets,
                      uint32_t* cids_new);

/* Rows in new-id order: out row n = X row inverse_perm[n] (dtype element
 * size x D bytes per row); data_reordered.<ext> (src/bucket.cu:9253-9400).
 * Also reorders any per-point table (e.g. vector_dists.bin rows as F32, D = M). */
int gt_permute_rows(gt_ctx* ctx, const void* X, int64_t N, int32_t D, int dtype, const uint32_t* inverse_perm,
                    void* out);

/* A per-point id table in new ids: out[n][k] = perm[ids[inverse_perm[n]][k]]
 * with perm the inverse permutation; ids outside [0, N) become -1 (the
 * vector_knn.bin of the reordered coordinate system). */
int gt_remap_table(gt_ctx* ctx, const int32_t* ids, int64_t N, int32_t M, const uint32_t* inverse_perm,
                   int32_t* out);

/* Beam (ef) search.  Defaults (gt_search_params_default) are the reference
 * CLI's: topk 10, ef 200, num_entry 4 (bd/search.py:280-283), L2, seed 42. */
typedef struct gt_search_params {
    int32_t topk;           /* results per query (--topk) */
    int32_t ef;             /* beam width (--ef), raised to topk as bd/search.py:164 does; <= 2048 */
    int32_t num_entry;      /* entry points per query drawn when `entries` is NULL (--num-entry), <= 64 */
    int32_t metric;         /* GT_METRIC_L2 (the reference's only metric) or GT_METRIC_IP */
    uint64_t seed;          /* entry draw when `entries` is NULL */
    int32_t visited_slots;  /* visited set per query: 0 = automatic (an on-chip hash table, or an HBM
                               bitmap of N bits per wave when the table would take more than 32 KiB
                               of LDS); -1 = the HBM bitmap; else the on-chip table's slots (power of
                               two >= 512), a query that outgrows it run again with the bitmap */
    int32_t reserved_;
} gt_search_params;

typedef struct gt_search_stats {
    double t_total;         /* wall seconds of the whole call */
    double t_search;        /* search kernels (device time) */
    int64_t expansions;     /* nodes popped and expanded, all queries */
    int64_t visited;        /* distances computed, all queries */
    int64_t requeued;       /* queries run a second time with the HBM bitmap */
} gt_search_stats;

void gt_search_params_default(gt_search_params* p);

/* Beam search of nq queries Q (nq x D, same dtype as X) over a graph
 * (N x degree ids; ids >= N, e.g. 0xFFFFFFFF padding, are skipped): per query
 * the sequential best-first search of bd/search.py:20-90
 * (graph_search_single) -- entry points in order, pop the smallest
 * (distance, id) candidate, stop when ef results are held and the popped
 * distance exceeds their maximum, a strictly closer point replaces the first
 * slot holding the maximum.  entries: (nq x n_entry) int32 entry points
 * (< 0 skipped), or NULL to draw params->num_entry per query (sorted,
 * distinct, seeded; not numpy's generator -- the Python mirror passes
 * numpy's draws).  out_ids / out_d: (nq x topk) ascending in distance, ties
 * in result-slot order, padded with -1 / +inf; with GT_METRIC_IP out_d is the
 * inner product (descending).  Replaces the per-query loop of
 * search_graph_recall (bd/search.py:165-174, bd/search.cpp:305-320). */
int gt_search(gt_ctx* ctx, const void* X, int64_t N, int32_t D, int dtype, const uint32_t* graph,
              int32_t degree, const void* Q, int64_t nq, const int32_t* entries, int32_t n_entry,
              const gt_search_params* params, int32_t* out_ids, float* out_d, gt_search_stats* stats);

/* Path selection of a context, for tests and A/B comparisons.  Every choice
 * gives the same results bit for bit; the defaults (gt_debug_opts_default)
 * take the fastest path for each shape.  The reference selects its
 * alternative paths with BUCKET2_* environment variables
 * (src/bucket.cu:5375, :5507); here they are a typed per-context setting. */
typedef struct gt_debug_opts {
    int32_t knn_collect;     /* 1 (default): collect + select kNN where it applies; 0: merging kernels */
    int32_t revmerge_path;   /* reverse merge: 0 (default) by shape, 1 two-kernel (where it applies),
                                2 binned, 3 global-atomic CSR, 4 two-kernel behind superbins */
    int32_t sub_order;       /* 1 (default): unseeded passes scan members by nearest sub-centroid;
                                0: the two-choice order */
    int32_t lloyd_host_csr;  /* 0 (default): Lloyd groups on the device; 1: on the host */
    int32_t prune_flat_rows; /* 0 (default): the prune fetches neighbour rows by buffer loads when the
                                table is below 2 GiB; 1: always the flat 64-bit addressing of larger
                                tables */
    int32_t knn_stats;       /* 1 with GTANN_TRACE set: per-launch counters of the collect kernel */
    int32_t knn_prune;       /* 1 (default): the int8 collect kernel skips pool chunks whose bounding
                                sphere is farther from every query than its threshold (exact); 0: scans all */
    int32_t bucket_host_csr; /* 0 (default): the bucket members are ordered on the device (the host
                                runs only the two-choice rule); 1: on the host (same order) */
    int32_t knn_resident;    /* 1 (default): short lists of int8 rows against a centroid set that fits
                                the LDS (top-2 assignment, Lloyd steps, probe tables; up to 512
                                centroids of 128 bytes) with the centroids held there; 0: the
                                staged-pool kernel */
    int32_t knn_window;      /* tiles of 32 pool rows in the unseeded collect pass's threshold window
                                (2..32, even); 0 (default): 32 on builds of 2^22 rows or more, else 16 */
    int32_t knn_screen;      /* 1 (default): collect passes on fp32 rows (Dp <= 160, pools of at most
                                32768 rows) of at least 2^27 (query, pool) pairs scan each work item's
                                pool on the fp16 matrix cores first (an unseeded pass also bounds its
                                thresholds there) and run the fp32 pass over the rows that can reach a
                                list (same tables bit for bit); 2: every such pass, whatever its size;
                                0: the fp32 pass over every pool row */
} gt_debug_opts;

void gt_debug_opts_default(gt_debug_opts* o);
/* Sets the context's options (NULL: the defaults). */
int gt_set_debug(gt_ctx* ctx, const gt_debug_opts* o);

#ifdef __cplusplus
}
#endif
#endif /* GTANN_H */
