/*
 * gt_oracle.c -- CPU restatement of the reference's bucketed CAGRA-style graph
 * build, used ONLY as test infrastructure: the parity checker for the HIP
 * library and the timed CPU baseline of bench.py.  Nothing in the shipped
 * library links, loads or calls this file.
 *
 * Every function cites the reference file:line it restates (paths relative
 * to loulankxh/GPU-talored-ANN, bd/ = bucketDemo/, src/ = bucketDemo/buildBucket/src/).
 *
 * Conventions shared with the HIP library:
 *   - a kNN row is ascending in (distance, id); padding is (-1, +inf);
 *   - L2 distances are squared Euclidean; for the inner-product metric the
 *     row key is -<x,y> (ascending key = descending similarity);
 *   - the oracle accumulates in double, so for integer-valued data with
 *     D*255^2 < 2^24 every distance is the exact integer the GPU also gets.
 *
 * Pinning of each function (what checks it other than itself) is listed in
 * the header of oracle/gt_oracle.py.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

#define OR_OK 0
#define OR_EINVAL (-1)
#define OR_ENOMEM (-2)
#define OR_EFEWCAND (-4)

typedef struct { double d; int32_t id; } cand_t;

static int cand_less(const cand_t* a, const cand_t* b)
{
    if (a->d < b->d) return 1;
    if (a->d > b->d) return 0;
    return a->id < b->id;
}

/* Bounded insertion into a sorted top-M list (ascending (d, id)). */
static void topm_insert(cand_t* list, int* n, int M, cand_t c)
{
    if (*n == M && !cand_less(&c, &list[M - 1])) return;
    int pos = (*n < M) ? (*n)++ : M - 1;
    while (pos > 0 && cand_less(&c, &list[pos - 1])) { list[pos] = list[pos - 1]; --pos; }
    list[pos] = c;
}

static double pair_key(const float* X, int64_t D, int64_t a, int64_t b, const double* norms, int metric)
{
    const float* xa = X + a * D;
    const float* xb = X + b * D;
    double dot = 0.0;
    for (int64_t k = 0; k < D; ++k) dot += (double)xa[k] * (double)xb[k];
    if (metric == 1) return -dot;
    return norms[a] + norms[b] - 2.0 * dot;
}

static double* row_norms(const float* X, int64_t N, int64_t D)
{
    double* n = (double*)malloc(sizeof(double) * (size_t)(N > 0 ? N : 1));
    if (!n) return NULL;
    #pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < N; ++i) {
        double s = 0.0;
        for (int64_t k = 0; k < D; ++k) s += (double)X[i * D + k] * (double)X[i * D + k];
        n[i] = s;
    }
    return n;
}

static void write_row(const cand_t* list, int n, int M, int32_t* ids, float* d)
{
    for (int k = 0; k < M; ++k) {
        ids[k] = k < n ? list[k].id : -1;
        d[k] = k < n ? (float)list[k].d : INFINITY;
    }
}

/*
 * Exact kNN of the queries qids[0..nq) against all N points.
 * Restates bd/build_knn.py:17-149 (self excluded, bd/build_knn.py:34-38;
 * dist = |a|^2 + |b|^2 - 2ab, bd/build_knn.py:31-32) with the tie rule
 * ascending (distance, id).  exclude_self = 0 keeps the query itself.
 */
int or_knn_exact(const float* X, int64_t N, int64_t D, int metric,
                 const int64_t* qids, int64_t nq, int M, int exclude_self,
                 int32_t* out_ids, float* out_d)
{
    if (!X || N <= 0 || D <= 0 || M <= 0 || nq < 0) return OR_EINVAL;
    double* norms = row_norms(X, N, D);
    if (!norms) return OR_ENOMEM;
    int err = 0;
    #pragma omp parallel
    {
        cand_t* list = (cand_t*)malloc(sizeof(cand_t) * (size_t)M);
        if (!list) {
            #pragma omp atomic write
            err = 1;
        }
        #pragma omp for schedule(dynamic, 4)
        for (int64_t qi = 0; qi < nq; ++qi) {
            if (!list) continue;
            int64_t q = qids[qi];
            int n = 0;
            for (int64_t p = 0; p < N; ++p) {
                if (exclude_self && p == q) continue;
                cand_t c = { pair_key(X, D, q, p, norms, metric), (int32_t)p };
                topm_insert(list, &n, M, c);
            }
            write_row(list, n, M, out_ids + qi * M, out_d + qi * M);
        }
        free(list);
    }
    free(norms);
    return err ? OR_ENOMEM : OR_OK;
}

/*
 * Pooled (bucketed) kNN of one round.  The pool of bucket b is its own
 * members followed by the members of its probe buckets, restating
 * src/bucket.cu:5331-5347 (segment table; probe ids >= nB are skipped) and
 * the per-query top-M of src/bucket.cu:4101-4265 (self excluded, row written
 * at the query's global id, padding -1/+inf).  Duplicate probe ids are
 * counted once.  Output rows are indexed by global id; rows of points in no
 * bucket stay (-1, +inf).
 */
int or_knn_bucketed(const float* X, int64_t N, int64_t D, int metric,
                    const int64_t* offsets, const int32_t* members, int64_t nB,
                    const int32_t* probe, int P, int M,
                    int32_t* out_ids, float* out_d)
{
    if (!X || N <= 0 || D <= 0 || M <= 0 || nB <= 0 || P < 0) return OR_EINVAL;
    double* norms = row_norms(X, N, D);
    if (!norms) return OR_ENOMEM;
    for (int64_t i = 0; i < N * M; ++i) { out_ids[i] = -1; out_d[i] = INFINITY; }
    int err = 0;
    #pragma omp parallel
    {
        cand_t* list = (cand_t*)malloc(sizeof(cand_t) * (size_t)M);
        int64_t* segs = (int64_t*)malloc(sizeof(int64_t) * (size_t)(P + 1));
        if (!list || !segs) {
            #pragma omp atomic write
            err = 1;
        }
        #pragma omp for schedule(dynamic, 1)
        for (int64_t b = 0; b < nB; ++b) {
            if (!list || !segs) continue;
            int ns = 0;
            segs[ns++] = b;
            for (int j = 0; j < P; ++j) {
                int64_t pb = probe[b * P + j];
                if (pb < 0 || pb >= nB) continue;
                int dup = 0;
                for (int s = 0; s < ns; ++s) dup |= (segs[s] == pb);
                if (!dup) segs[ns++] = pb;
            }
            for (int64_t qi = offsets[b]; qi < offsets[b + 1]; ++qi) {
                int64_t q = members[qi];
                int n = 0;
                for (int s = 0; s < ns; ++s) {
                    for (int64_t pi = offsets[segs[s]]; pi < offsets[segs[s] + 1]; ++pi) {
                        int64_t p = members[pi];
                        if (p == q) continue;
                        cand_t c = { pair_key(X, D, q, p, norms, metric), (int32_t)p };
                        topm_insert(list, &n, M, c);
                    }
                }
                write_row(list, n, M, out_ids + q * M, out_d + q * M);
            }
        }
        free(list);
        free(segs);
    }
    free(norms);
    return err ? OR_ENOMEM : OR_OK;
}

/*
 * Cross-round merge: top-M by (distance, id) of run U new, an id present in
 * both taken once (with the running distance).  Restates the intent of
 * src/bucket.cu:5021-5053 (two ascending lists, new ids already in the
 * running list skipped, padded -1/+inf); ties are ordered by id instead of
 * "running first" so the result does not depend on the round order.
 */
int or_merge_rounds(const int32_t* run_ids, const float* run_d,
                    const int32_t* new_ids, const float* new_d,
                    int64_t N, int M, int32_t* out_ids, float* out_d)
{
    if (N < 0 || M <= 0) return OR_EINVAL;
    int err = 0;
    #pragma omp parallel
    {
        cand_t* list = (cand_t*)malloc(sizeof(cand_t) * (size_t)M);
        if (!list) {
            #pragma omp atomic write
            err = 1;
        }
        #pragma omp for schedule(static)
        for (int64_t i = 0; i < N; ++i) {
            if (!list) continue;
            int n = 0;
            const int32_t* a = run_ids + i * M;
            const int32_t* b = new_ids + i * M;
            for (int k = 0; k < M; ++k) {
                if (a[k] < 0) continue;
                cand_t c = { run_d[i * M + k], a[k] };
                topm_insert(list, &n, M, c);
            }
            for (int k = 0; k < M; ++k) {
                if (b[k] < 0) continue;
                int dup = 0;
                for (int t = 0; t < M; ++t) dup |= (a[t] == b[k]);
                if (dup) continue;
                cand_t c = { new_d[i * M + k], b[k] };
                topm_insert(list, &n, M, c);
            }
            write_row(list, n, M, out_ids + i * M, out_d + i * M);
        }
        free(list);
    }
    return err ? OR_ENOMEM : OR_OK;
}

/*
 * Sanitize: -1 / out-of-range / self entries become the row's first valid
 * neighbour, else (i+1) % N; output as uint32.  Restates
 * src/optimize.cu:89-134 (and src/bucket.cu:8444-8463).  Returns the number
 * of replaced -1 entries.
 */
int64_t or_sanitize(const int32_t* knn, int64_t N, int M, uint32_t* out)
{
    int64_t padding = 0;
    #pragma omp parallel for schedule(static) reduction(+:padding)
    for (int64_t i = 0; i < N; ++i) {
        const int32_t* row = knn + i * M;
        uint32_t fallback = (uint32_t)((i + 1) % N);
        for (int j = 0; j < M; ++j) {
            int32_t v = row[j];
            if (v >= 0 && v < N && (int64_t)v != i) { fallback = (uint32_t)v; break; }
        }
        for (int j = 0; j < M; ++j) {
            int32_t v = row[j];
            if (v < 0 || v >= N || (int64_t)v == i) {
                out[i * M + j] = fallback;
                if (v < 0) padding++;
            } else {
                out[i * M + j] = (uint32_t)v;
            }
        }
    }
    return padding;
}

/*
 * CAGRA detour counts of one point, full window.  Restates
 * src/prune_windowed_core.hpp:189-232: count[kAB] = #{kAD < kAB :
 * row[kAD] is a valid point id and row[kAB] occurs in row(row[kAD])}, each
 * (kAD, kAB) pair counted at most once, duplicate ids in the row kept as
 * separate ranks.  Entries are int32 (-1 = padding); a detour source D must
 * lie in [0, N) (src/prune_windowed_core.hpp:102-103,217).
 */
static int cmp_i32(const void* x, const void* y)
{
    int32_t a = *(const int32_t*)x, b = *(const int32_t*)y;
    return (a > b) - (a < b);
}

/* Bucket windows (src/prune_windowed_core.hpp:77-124 BucketWindow): ids are
 * bucket-contiguous, position q owning [off[q], off[q+1]); row a's window is
 * the positions win[p*W .. p*W + win_len[p]) of a's own position p.  NULL
 * off: every row is visible (the full prune). */
typedef struct {
    const uint32_t* off;
    int nb;
    const int32_t* win;
    const int32_t* win_len;
    int W;
} window_t;

static int pos_of(const window_t* w, uint32_t id)   /* last q with off[q] <= id */
{
    int lo = 0, hi = w->nb - 1;
    while (lo < hi) {
        int mid = (lo + hi + 1) / 2;
        if (w->off[mid] <= id) lo = mid;
        else hi = mid - 1;
    }
    return lo;
}

static int visible(const window_t* w, int64_t a, int32_t d)
{
    if (!w || !w->off) return 1;
    int p = pos_of(w, (uint32_t)a), q = pos_of(w, (uint32_t)d);
    for (int i = 0; i < w->win_len[p]; ++i)
        if (w->win[(int64_t)p * w->W + i] == q) return 1;
    return 0;
}

static void detour_counts_w(const int32_t* G, int64_t N, int M, int64_t a, uint32_t* count, const window_t* win)
{
    const int32_t* A = G + a * M;
    int32_t drow[512];   /* M <= 512: the row of D, sorted for membership tests */
    for (int k = 0; k < M; ++k) count[k] = 0;
    for (int kAD = 0; kAD < M - 1; ++kAD) {
        int32_t d = A[kAD];
        if (d < 0 || (int64_t)d >= N) continue;
        if (!visible(win, a, d)) continue;   /* outside the window: contributes nothing */
        memcpy(drow, G + (int64_t)d * M, sizeof(int32_t) * (size_t)M);
        qsort(drow, (size_t)M, sizeof(int32_t), cmp_i32);
        for (int kAB = kAD + 1; kAB < M; ++kAB) {
            int32_t b = A[kAB];
            if (b < 0) continue;
            if (bsearch(&b, drow, (size_t)M, sizeof(int32_t), cmp_i32)) count[kAB]++;
        }
    }
}

static void detour_counts(const int32_t* G, int64_t N, int M, int64_t a, uint32_t* count)
{
    detour_counts_w(G, N, M, a, count, NULL);
}

/*
 * CAGRA rank-based prune: rows are already in rank order (no L2 re-sort),
 * detour counts as above, then the first K valid candidates in
 * (count, rank) order.  Restates src/prune_windowed_core.hpp:238-263
 * (select_pruned_row).  Returns OR_EFEWCAND (reporting the first offending
 * row in *bad_row) when a row has fewer than K valid candidates
 * (src/prune_windowed_core.hpp:257-260).
 */
static int cagra_prune_w(const int32_t* G, int64_t N, int M, int K, uint32_t* out, int64_t* bad_row,
                         const window_t* win)
{
    if (!G || N <= 0 || M <= 0 || M > 512 || K <= 0 || K > M) return OR_EINVAL;
    int64_t first_bad = -1;
    #pragma omp parallel
    {
        uint32_t* cnt = (uint32_t*)malloc(sizeof(uint32_t) * (size_t)M);
        #pragma omp for schedule(dynamic, 64)
        for (int64_t a = 0; a < N; ++a) {
            const int32_t* A = G + a * M;
            detour_counts_w(G, N, M, a, cnt, win);
            int pk = 0;
            uint32_t level = 0;
            while (pk < K) {
                uint32_t next = UINT32_MAX;
                for (int k = 0; k < M && pk < K; ++k) {
                    if (A[k] < 0) continue;
                    if (cnt[k] > level && cnt[k] < next) next = cnt[k];
                    if (cnt[k] != level) continue;
                    out[a * K + pk++] = (uint32_t)A[k];
                }
                if (pk >= K) break;
                if (next == UINT32_MAX) {
                    #pragma omp critical
                    { if (first_bad < 0 || a < first_bad) first_bad = a; }
                    break;
                }
                level = next;
            }
        }
        free(cnt);
    }
    if (bad_row) *bad_row = first_bad;
    return first_bad >= 0 ? OR_EFEWCAND : OR_OK;
}

int or_cagra_prune(const int32_t* G, int64_t N, int M, int K, uint32_t* out, int64_t* bad_row)
{
    return cagra_prune_w(G, N, M, K, out, bad_row, NULL);
}

/*
 * Windowed CAGRA prune (src/prune_windowed_core.hpp:177-263 with a
 * BucketWindow per processing position, src/prune_windowed.cpp:300-420;
 * src/prune_windowed_gpu.cu:181-326): as or_cagra_prune, but a detour
 * through D counts only when D's bucket position is in the window of the
 * pruned row's position.  Rows are taken in the given (rank) order.
 */
int or_prune_windowed(const int32_t* G, int64_t N, int M, const uint32_t* off, int nb, const int32_t* win,
                      const int32_t* win_len, int W, int K, uint32_t* out, int64_t* bad_row)
{
    if (!off || nb <= 0 || off[0] != 0 || (int64_t)off[nb] != N || !win || !win_len || W <= 0) return OR_EINVAL;
    window_t w = {off, nb, win, win_len, W};
    return cagra_prune_w(G, N, M, K, out, bad_row, &w);
}

/* detour counts exported for the known-answer tests */
int or_detour_counts(const int32_t* G, int64_t N, int M, int64_t a, uint32_t* count)
{
    if (!G || a < 0 || a >= N || M > 512) return OR_EINVAL;
    detour_counts(G, N, M, a, count);
    return OR_OK;
}

typedef struct { uint32_t rank; uint32_t src; } rev_t;

static int rev_cmp(const void* x, const void* y)
{
    const rev_t* a = (const rev_t*)x;
    const rev_t* b = (const rev_t*)y;
    if (a->rank != b->rank) return a->rank < b->rank ? -1 : 1;
    if (a->src != b->src) return a->src < b->src ? -1 : 1;
    return 0;
}

/*
 * Reverse-edge merge (Method E).  Every forward edge (i, k) becomes a
 * reverse edge {dst = fwd[i][k], src = i, rank = k}
 * (src/optimize_chunked.cu:372-407); per dst the sources are ordered by
 * (rank, src) (src/edge_chunk_accumulator.hpp:235-284) and inserted weakest
 * first into the dst's own forward row, the first K/2 slots protected
 * (src/edge_chunk_accumulator.hpp:471-494, src/optimize_chunked.cu:1449-1471).
 * Returns OR_EINVAL if an edge points outside [0, N).
 */
int or_reverse_merge(const uint32_t* fwd, int64_t N, int K, uint32_t* out)
{
    if (!fwd || N <= 0 || K <= 0) return OR_EINVAL;
    int64_t E = N * K;
    uint32_t* deg = (uint32_t*)calloc((size_t)N + 1, sizeof(uint32_t));
    rev_t* recs = (rev_t*)malloc(sizeof(rev_t) * (size_t)(E > 0 ? E : 1));
    uint32_t* cur = (uint32_t*)malloc(sizeof(uint32_t) * (size_t)N);
    if (!deg || !recs || !cur) { free(deg); free(recs); free(cur); return OR_ENOMEM; }
    for (int64_t e = 0; e < E; ++e) {
        if (fwd[e] >= (uint64_t)N) { free(deg); free(recs); free(cur); return OR_EINVAL; }
        deg[fwd[e] + 1]++;
    }
    for (int64_t j = 0; j < N; ++j) deg[j + 1] += deg[j];
    memcpy(cur, deg, sizeof(uint32_t) * (size_t)N);
    for (int64_t i = 0; i < N; ++i)
        for (int k = 0; k < K; ++k) {
            uint32_t j = fwd[i * K + k];
            rev_t r = { (uint32_t)k, (uint32_t)i };
            recs[cur[j]++] = r;
        }
    const uint32_t P = (uint32_t)K / 2;
    #pragma omp parallel for schedule(dynamic, 256)
    for (int64_t j = 0; j < N; ++j) {
        uint32_t lo = deg[j], hi = deg[j + 1];
        qsort(recs + lo, hi - lo, sizeof(rev_t), rev_cmp);
        uint32_t* row = out + j * K;
        memcpy(row, fwd + j * K, sizeof(uint32_t) * (size_t)K);
        for (uint32_t k = hi; k > lo;) {
            --k;
            uint32_t s = recs[k].src;
            uint32_t pos = (uint32_t)K;
            for (uint32_t p = 0; p < (uint32_t)K; ++p) if (row[p] == s) { pos = p; break; }
            if (pos < P) continue;
            uint32_t shift = (pos == (uint32_t)K) ? ((uint32_t)K - P - 1) : (pos - P);
            for (uint32_t t = shift; t > 0; --t) row[P + t] = row[P + t - 1];
            row[P] = s;
        }
    }
    free(deg); free(recs); free(cur);
    return OR_OK;
}

/* merge_rank_ordered_into_row on one row, for the known-answer tests
 * (src/edge_chunk_accumulator.hpp:471-494). */
void or_merge_row(uint32_t* row, const uint32_t* rank_sorted_src, uint32_t count, uint32_t K)
{
    const uint32_t P = K / 2;
    for (uint32_t k = count; k > 0;) {
        --k;
        uint32_t s = rank_sorted_src[k];
        uint32_t pos = K;
        for (uint32_t p = 0; p < K; ++p) if (row[p] == s) { pos = p; break; }
        if (pos < P) continue;
        uint32_t shift = (pos == K) ? (K - P - 1) : (pos - P);
        for (uint32_t t = shift; t > 0; --t) row[P + t] = row[P + t - 1];
        row[P] = s;
    }
}

/*
 * 2-hop "pull" local-join refinement, one pass (reads in_*, writes out_*).
 * Restates src/bucket.cu:4754-4850 (a1_pull_join_kernel): candidates are the
 * first S neighbours of the first S neighbours; invalid, self and ids
 * already in the row are dropped; a candidate survives if its exact distance
 * is < the row's M-th distance; candidates are deduplicated; the new row is
 * the first M of row U survivors in (distance, id) order.
 */
int or_refine_2hop(const float* X, int64_t N, int64_t D, int metric,
                   const int32_t* in_ids, const float* in_d, int M, int S,
                   int32_t* out_ids, float* out_d)
{
    if (!X || N <= 0 || D <= 0 || M <= 0 || S <= 0 || S > M) return OR_EINVAL;
    double* norms = row_norms(X, N, D);
    if (!norms) return OR_ENOMEM;
    int err = 0;
    #pragma omp parallel
    {
        cand_t* list = (cand_t*)malloc(sizeof(cand_t) * (size_t)M);
        int32_t* seen = (int32_t*)malloc(sizeof(int32_t) * (size_t)S * (size_t)S);
        if (!list || !seen) {
            #pragma omp atomic write
            err = 1;
        }
        #pragma omp for schedule(dynamic, 64)
        for (int64_t a = 0; a < N; ++a) {
            if (!list || !seen) continue;
            const int32_t* row = in_ids + a * M;
            const double kth = in_d[a * M + M - 1];
            int n = 0, ns = 0;
            for (int k = 0; k < M; ++k) {
                if (row[k] < 0) continue;
                cand_t c = { in_d[a * M + k], row[k] };
                topm_insert(list, &n, M, c);
            }
            for (int c = 0; c < S * S; ++c) {
                int32_t u = row[c / S];
                if (u < 0 || u >= N) continue;
                int32_t v = in_ids[(int64_t)u * M + (c % S)];
                if (v < 0 || v >= N || v == a) continue;
                int dup = 0;
                for (int k = 0; k < M && !dup; ++k) dup = (row[k] == v);
                for (int t = 0; t < ns && !dup; ++t) dup = (seen[t] == v);
                if (dup) continue;
                seen[ns++] = v;
                double dv = pair_key(X, D, a, v, norms, metric);
                /* the reference compares the fp32 distance against kth */
                if (!((float)dv < (float)kth)) continue;
                cand_t cc = { (float)dv, v };
                topm_insert(list, &n, M, cc);
            }
            write_row(list, n, M, out_ids + a * M, out_d + a * M);
        }
        free(list);
        free(seen);
    }
    free(norms);
    return err ? OR_ENOMEM : OR_OK;
}

/*
 * Id translation: final[inv[i]][k] = inv[g[i][k]]; inv must be a
 * permutation.  Restates src/translate_graph_ids.hpp:75 and
 * src/optimize_chunked.cu:1493-1546.
 */
int or_translate(const uint32_t* g, const uint32_t* inv, int64_t N, int K, uint32_t* out)
{
    uint8_t* hit = (uint8_t*)calloc((size_t)N, 1);
    if (!hit) return OR_ENOMEM;
    for (int64_t i = 0; i < N; ++i) {
        uint32_t r = inv[i];
        if (r >= (uint64_t)N || hit[r]) { free(hit); return OR_EINVAL; }
        hit[r] = 1;
        for (int k = 0; k < K; ++k) {
            uint32_t v = g[i * K + k];
            if (v >= (uint64_t)N) { free(hit); return OR_EINVAL; }
            out[(int64_t)r * K + k] = inv[v];
        }
    }
    free(hit);
    return OR_OK;
}

typedef struct { float d; int32_t pos; int32_t id; } occ_t;

static int occ_cmp(const void* x, const void* y)
{
    const occ_t* a = (const occ_t*)x;
    const occ_t* b = (const occ_t*)y;
    if (a->d < b->d) return -1;
    if (a->d > b->d) return 1;
    return a->pos < b->pos ? -1 : (a->pos > b->pos);
}

static float l2_f32(const float* a, const float* b, int64_t D)
{
    double s = 0.0;
    for (int64_t k = 0; k < D; ++k) { double t = (double)a[k] - (double)b[k]; s += t * t; }
    return (float)s;
}

/*
 * Occlusion prune of bd/prune.py:8-83 (prune_graph): drop -1 / out-of-range /
 * self; sort by d(v, .) (ties by original column); z is removed when an
 * earlier kept u has d(u, z) < d(v, z); keep the first max_degree; pad -1.
 */
int or_prune_occlusion(const float* X, int64_t N, int64_t D, const int64_t* nb, int M,
                       int max_degree, int64_t* out)
{
    if (!X || !nb || N <= 0 || M <= 0) return OR_EINVAL;
    #pragma omp parallel
    {
        occ_t* c = (occ_t*)malloc(sizeof(occ_t) * (size_t)M);
        uint8_t* removed = (uint8_t*)malloc((size_t)M);
        #pragma omp for schedule(dynamic, 64)
        for (int64_t v = 0; v < N; ++v) {
            int n = 0;
            for (int k = 0; k < M; ++k) {
                int64_t z = nb[v * M + k];
                if (z < 0 || z >= N || z == v) continue;
                c[n].d = l2_f32(X + z * D, X + v * D, D);
                c[n].pos = k;
                c[n].id = (int32_t)z;
                ++n;
            }
            qsort(c, (size_t)n, sizeof(occ_t), occ_cmp);
            memset(removed, 0, (size_t)M);
            for (int i = 0; i < n; ++i) {
                if (removed[i]) continue;
                for (int j = i + 1; j < n; ++j) {
                    if (removed[j]) continue;
                    if (l2_f32(X + (int64_t)c[i].id * D, X + (int64_t)c[j].id * D, D) < c[j].d)
                        removed[j] = 1;
                }
            }
            int w = 0;
            for (int i = 0; i < n; ++i) {
                if (removed[i]) continue;
                if (max_degree > 0 && w >= max_degree) break;
                out[v * M + w++] = c[i].id;
            }
            for (; w < M; ++w) out[v * M + w] = -1;
        }
        free(c);
        free(removed);
    }
    return OR_OK;
}

/*
 * Reverse-edge insertion of bd/build_bucket.py:473-543 (_apply_reverse_edges),
 * in place on an N x M table whose rows are ascending.  All offers are taken
 * from the table as it was on entry (:485-492).  Edge a -> b (distance d, from
 * a's row) is offered to b when d < max(b's row) (the per-target skip at
 * :517-519 keeps exactly these); offers whose source is already in b's row are
 * dropped (:522-524); repeated offers are kept (:527-529).  A row with a
 * surviving offer becomes the first M of (row, offers) in (distance, id)
 * order, ids compared as unsigned so -1 padding sorts last among equal
 * distances (torch.topk's order among ties, :533, is not specified; this
 * order is ours).  Returns OR_EINVAL if an id is >= N.
 */
typedef struct { float d; uint32_t id; } rin_t;

static int rin_cmp(const void* x, const void* y)
{
    const rin_t* a = (const rin_t*)x;
    const rin_t* b = (const rin_t*)y;
    if (a->d < b->d) return -1;
    if (a->d > b->d) return 1;
    return a->id < b->id ? -1 : (a->id > b->id);
}

int or_reverse_insert(int32_t* ids, float* d, int64_t N, int M)
{
    if (!ids || !d || N <= 0 || M <= 0) return OR_EINVAL;
    const int64_t E = N * M;
    for (int64_t e = 0; e < E; ++e)
        if (ids[e] >= N) return OR_EINVAL;
    float* worst = (float*)malloc(sizeof(float) * (size_t)N);
    int64_t* off = (int64_t*)calloc((size_t)N + 1, sizeof(int64_t));
    for (int64_t b = 0; b < N; ++b) {
        float w = -INFINITY;
        for (int k = 0; k < M; ++k) w = fmaxf(w, d[b * M + k]);
        worst[b] = w;
    }
    for (int64_t e = 0; e < E; ++e)
        if (ids[e] >= 0 && d[e] < worst[ids[e]]) off[ids[e] + 1]++;
    for (int64_t b = 0; b < N; ++b) off[b + 1] += off[b];
    rin_t* offers = (rin_t*)malloc(sizeof(rin_t) * (size_t)(off[N] + 1));
    int64_t* fill = (int64_t*)malloc(sizeof(int64_t) * (size_t)N);
    memcpy(fill, off, sizeof(int64_t) * (size_t)N);
    for (int64_t e = 0; e < E; ++e) {
        const int32_t b = ids[e];
        if (b >= 0 && d[e] < worst[b]) {
            offers[fill[b]].d = d[e];
            offers[fill[b]].id = (uint32_t)(e / M);
            fill[b]++;
        }
    }
    int32_t* new_ids = (int32_t*)malloc(sizeof(int32_t) * (size_t)E);
    float* new_d = (float*)malloc(sizeof(float) * (size_t)E);
    memcpy(new_ids, ids, sizeof(int32_t) * (size_t)E);
    memcpy(new_d, d, sizeof(float) * (size_t)E);
    #pragma omp parallel
    {
        rin_t* buf = NULL;
        int64_t cap = 0;
        #pragma omp for schedule(dynamic, 256)
        for (int64_t b = 0; b < N; ++b) {
            const int64_t n = off[b + 1] - off[b];
            if (n == 0) continue;
            if (n + M > cap) { cap = n + M; buf = (rin_t*)realloc(buf, sizeof(rin_t) * (size_t)cap); }
            int64_t cnt = 0;
            for (int k = 0; k < M; ++k) { buf[cnt].d = d[b * M + k]; buf[cnt].id = (uint32_t)ids[b * M + k]; ++cnt; }
            int64_t added = 0;
            for (int64_t t = off[b]; t < off[b + 1]; ++t) {
                int in_row = 0;
                for (int k = 0; k < M; ++k) in_row |= (uint32_t)ids[b * M + k] == offers[t].id;
                if (!in_row) { buf[cnt++] = offers[t]; ++added; }
            }
            if (added == 0) continue;
            qsort(buf, (size_t)cnt, sizeof(rin_t), rin_cmp);
            for (int k = 0; k < M; ++k) { new_ids[b * M + k] = (int32_t)buf[k].id; new_d[b * M + k] = buf[k].d; }
        }
        free(buf);
    }
    memcpy(ids, new_ids, sizeof(int32_t) * (size_t)E);
    memcpy(d, new_d, sizeof(float) * (size_t)E);
    free(worst); free(off); free(offers); free(fill); free(new_ids); free(new_d);
    return OR_OK;
}

int or_num_threads(void)
{
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}

/* ------------------------------------------------------------------ search
 * Beam (ef) search over a graph, one query at a time, as
 * bd/search.py:20-90 (graph_search_single):
 *   - entry points in the given order (the Python pipeline passes
 *     np.unique(rng.integers(0, N, num_entry)), bd/search.py:41-42), each
 *     visited and inserted like a neighbour (:43-54);
 *   - pop the candidate with the smallest (distance, id) -- heapq's tuple
 *     order (:56-57); stop when the best list holds ef points and the popped
 *     distance exceeds its maximum (:58-62);
 *   - expand the popped node's row in order, skipping ids outside [0, N)
 *     and visited ones (:64-71); every newly visited point becomes a
 *     candidate (:72);
 *   - the best list is an array of at most ef slots: append while short,
 *     else a strictly closer point replaces the first slot holding the
 *     maximum (np.argmax, :74-81);
 *   - output: the best list sorted by distance with ties in slot order (a
 *     stable argsort; the reference's np.argsort is numpy's unstable sort,
 *     :87-89), first topk, padded with (-1, +inf) (:171-174).
 * Distances: sum over dims of (q - x)^2 (bd/search.py:12-14 l2sqr), or
 * -sum q*x for the inner product, as four fmaf partial sums by dimension
 * mod 4 combined as (s0 + s1) + (s2 + s3) -- the GPU kernel's order (the
 * reference's own order is its BLAS's).
 */
typedef struct { float d; uint32_t id; } sc_t;

static int sc_less(sc_t a, sc_t b) { return a.d < b.d || (a.d == b.d && a.id < b.id); }

static void sc_push(sc_t* h, int64_t* n, sc_t x)
{
    int64_t i = (*n)++;
    while (i > 0) {
        const int64_t p = (i - 1) / 2;
        if (!sc_less(x, h[p])) break;
        h[i] = h[p];
        i = p;
    }
    h[i] = x;
}

static sc_t sc_pop(sc_t* h, int64_t* n)
{
    const sc_t top = h[0];
    const sc_t x = h[--(*n)];
    int64_t i = 0;
    for (;;) {
        int64_t c = 2 * i + 1;
        if (c >= *n) break;
        if (c + 1 < *n && sc_less(h[c + 1], h[c])) ++c;
        if (!sc_less(h[c], x)) break;
        h[i] = h[c];
        i = c;
    }
    if (*n > 0) h[i] = x;
    return top;
}

static float search_dist(const float* q, const float* x, int64_t D, int metric)
{
    /* four partial sums by dimension mod 4, combined as (s0 + s1) + (s2 + s3) */
    float s[4] = {0.f, 0.f, 0.f, 0.f};
    for (int64_t k = 0; k < D; ++k) {
        if (metric == 1) {
            s[k & 3] = fmaf(q[k], x[k], s[k & 3]);
        } else {
            const float t = q[k] - x[k];
            s[k & 3] = fmaf(t, t, s[k & 3]);
        }
    }
    const float r = (s[0] + s[1]) + (s[2] + s[3]);
    return metric == 1 ? -r : r;
}

int or_search(const float* X, int64_t N, int64_t D, const uint32_t* graph, int deg, const float* Q, int64_t nq,
              const int32_t* entries, int n_entry, int topk, int ef, int metric, int32_t* out_ids, float* out_d,
              int64_t* expansions)
{
    if (N <= 0 || D <= 0 || deg < 0 || n_entry < 1 || topk < 1 || ef < topk) return OR_EINVAL;
    int err = OR_OK;
    #pragma omp parallel
    {
        uint8_t* seen = (uint8_t*)calloc((size_t)N, 1);
        int64_t hcap = 1024, vcap = 1024;
        sc_t* heap = (sc_t*)malloc(sizeof(sc_t) * (size_t)hcap);
        uint32_t* vis = (uint32_t*)malloc(sizeof(uint32_t) * (size_t)vcap);
        float* bd = (float*)malloc(sizeof(float) * (size_t)ef);
        uint32_t* bi = (uint32_t*)malloc(sizeof(uint32_t) * (size_t)ef);
        int* ord = (int*)malloc(sizeof(int) * (size_t)ef);
        if (!seen || !heap || !vis || !bd || !bi || !ord) {
            #pragma omp atomic write
            err = OR_ENOMEM;
        }
        #pragma omp for schedule(dynamic, 4)
        for (int64_t qi = 0; qi < nq; ++qi) {
            if (err) continue;
            const float* q = Q + qi * D;
            int64_t nh = 0, nv = 0, nexp = 0;
            int nb = 0;
            /* visit v: mark, distance, candidate, best list (bd/search.py:70-81) */
#define OR_VISIT(vv)                                                                                  \
            do {                                                                                      \
                const uint32_t v_ = (vv);                                                             \
                seen[v_] = 1;                                                                         \
                if (nv == vcap) { vcap *= 2; vis = (uint32_t*)realloc(vis, sizeof(uint32_t) * (size_t)vcap); } \
                vis[nv++] = v_;                                                                       \
                const float dv_ = search_dist(q, X + (int64_t)v_ * D, D, metric);                     \
                if (nh == hcap) { hcap *= 2; heap = (sc_t*)realloc(heap, sizeof(sc_t) * (size_t)hcap); } \
                sc_t c_ = {dv_, v_};                                                                  \
                sc_push(heap, &nh, c_);                                                               \
                if (nb < ef) { bd[nb] = dv_; bi[nb] = v_; ++nb; }                                     \
                else {                                                                                \
                    int w_ = 0;                                                                       \
                    for (int t_ = 1; t_ < nb; ++t_) if (bd[t_] > bd[w_]) w_ = t_;                     \
                    if (dv_ < bd[w_]) { bd[w_] = dv_; bi[w_] = v_; }                                  \
                }                                                                                     \
            } while (0)
            for (int e = 0; e < n_entry; ++e) {
                const int32_t s = entries[qi * n_entry + e];
                if (s < 0 || s >= N || seen[s]) continue;
                OR_VISIT((uint32_t)s);
            }
            while (nh > 0) {
                const sc_t u = sc_pop(heap, &nh);
                if (nb >= ef) {
                    float worst = bd[0];
                    for (int t = 1; t < nb; ++t) worst = bd[t] > worst ? bd[t] : worst;
                    if (u.d > worst) break;
                }
                ++nexp;
                const uint32_t* row = graph + (int64_t)u.id * deg;
                for (int j = 0; j < deg; ++j) {
                    const uint32_t v = row[j];
                    if (v >= (uint64_t)N || seen[v]) continue;
                    OR_VISIT(v);
                }
            }
#undef OR_VISIT
            /* stable order of the best list by distance */
            for (int t = 0; t < nb; ++t) ord[t] = t;
            for (int t = 1; t < nb; ++t) {
                const int x = ord[t];
                int p = t;
                while (p > 0 && bd[ord[p - 1]] > bd[x]) { ord[p] = ord[p - 1]; --p; }
                ord[p] = x;
            }
            for (int t = 0; t < topk; ++t) {
                out_ids[qi * topk + t] = t < nb ? (int32_t)bi[ord[t]] : -1;
                out_d[qi * topk + t] = t < nb ? bd[ord[t]] : INFINITY;
            }
            if (expansions) expansions[qi] = nexp;
            for (int64_t t = 0; t < nv; ++t) seen[vis[t]] = 0;
        }
        free(seen); free(heap); free(vis); free(bd); free(bi); free(ord);
    }
    return err;
}

/* ------------------------------------------------------------- bucket reorder
 * compute_bucket_reorder (src/bucket.cu:8363-8412): bucket b's range of new
 * ids starts after the points of every bucket placed before it in `order`;
 * old ids are dealt in increasing order to their bucket's next new id.
 * inverse_perm[new] = old, offsets[pos + 1] = end of position pos's range.
 * Points without a bucket in [0, nb) are skipped (the reference counts them
 * as unassigned); returns the number placed.
 */
int64_t or_bucket_reorder(const int32_t* assign, int64_t N, int64_t nb, const int32_t* order, uint32_t* inverse_perm,
                          uint32_t* offsets)
{
    int64_t* count = (int64_t*)calloc((size_t)nb, sizeof(int64_t));
    uint32_t* cursor = (uint32_t*)malloc(sizeof(uint32_t) * (size_t)nb);
    if (!count || !cursor) { free(count); free(cursor); return OR_ENOMEM; }
    for (int64_t i = 0; i < N; ++i)
        if (assign[i] >= 0 && assign[i] < nb) count[assign[i]]++;
    uint32_t run = 0;
    offsets[0] = 0;
    for (int64_t q = 0; q < nb; ++q) {
        cursor[order[q]] = run;
        run += (uint32_t)count[order[q]];
        offsets[q + 1] = run;
    }
    for (int64_t i = 0; i < N; ++i)
        if (assign[i] >= 0 && assign[i] < nb) inverse_perm[cursor[assign[i]]++] = (uint32_t)i;
    free(count);
    free(cursor);
    return (int64_t)run;
}
