// gtann_main.cpp -- command-line front end of libgtann.so, one subcommand per
// executable of the reference pipeline (sk/scripts/run_pipeline.sh:111-148):
//
//   gtann bucket2 -i BASE -o OUT [--centroid-ratio R] [--seed S] [--knn-k K]
//         [--nprobe P] [--neighbors-m M] [-t T] [--fused-optimize-degree K]
//         [--order-window W] [--skip-dists] [--skip-npy] [--kmeans-iters I]
//         [--balance F] [--refine-passes P] [--refine-sample S] [--gpu-limit BYTES]
//       the GPU-resident build (src/bucket.cu:9900-9990 options) with the
//       inline reorder of round 1 (src/bucket.cu:9160-9460): new ids are
//       bucket-contiguous, buckets in the DiskJoin order of the round-1
//       centroid kNN graph.  Writes, under OUT/k<knn-k>p<nprobe>m<M>t<T>/
//       (src/bucket.cu:8545-8556): data_reordered<ext>, inverse_perm.bin,
//       bucket_offsets.bin, bucket_process_order.bin, centroid_knn.bin,
//       centroid_pool.bin (with --nprobe), vector_knn.bin, vector_dists.bin
//       and neighbors.npy in new ids, and with --fused-optimize-degree K > 0
//       final_graph.bin in the input's ids.  --gpu-limit below the tables:
//       the out-of-core build (running table in host memory, chunked), same
//       files.
//   gtann optimize -i DATA -g KNN -o OUT --output-degree K [--skip-sort]
//       sanitize + CAGRA prune + reverse merge (src/optimize.cu); exit 2 when
//       the device cannot hold the tables (the reference's "use the other
//       path" code, src/optimize.cu:300-308).
//   gtann prune_windowed -k KNN -i DATA -o FWD --output-degree K
//         [--bucket-offsets F --bucket-process-order F -c CENTROID_KNN] [--pool-graph F]
//         [--cache-mb MB]
//       the windowed CAGRA prune (src/prune_windowed.cpp): each bucket's rows
//       see only the rows of the buckets in its window, positions chunked
//       within --cache-mb of device memory; without the bucket files,
//       sanitize + the full prune.
//   gtann optimize_chunked -g FWD -o OUT [-m E] [--gpu-budget-mb MB]
//         [--inverse-perm P --final-output F]
//       reverse-edge merge (Method E), in destination chunks when the graph
//       exceeds --gpu-budget-mb, optionally translated to original ids.
//   gtann translate_ids -g G -p P -o OUT
//       out[inv[i]][k] = inv[g[i][k]] (src/translate_ids.cpp).
//   gtann knn -i DATA -o OUTDIR -k K
//       exact self-excluded kNN (bd/build_knn.py) as vector_knn.bin/vector_dists.bin.
//   gtann search --base B --query Q --index IDX --gt GT [--topk 10] [--ef 200]
//         [--num-entry 4] [--normalize]
//       beam search of every query and recall against the ground truth, as
//       bd/search.cpp's `search` (options, file readers, entry draw with
//       std::mt19937(42), recall definitions and report lines); the search
//       itself is gt_search.  IDX: .npy (int64/int32/uint32) or a graph .bin.
//   gtann compare --index1 A --index2 B [--k-cmp K] [--save-csv F]
//       set-wise comparison of two indices (bd/search.cpp compare, with the
//       per-node CSV of bd/search.py:238-262).
//
// The reference's device budgets (--gpu-limit, --cache-mb, --gpu-budget-mb)
// select the out-of-core stages; its other options that tune host memory,
// disk buffers or its own caches are accepted and ignored.  Errors print
// "FATAL: <message>" and exit 1.
#include "gtann.h"
#include "gtann_io.hpp"

#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <chrono>
#include <random>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <map>
#include <set>
#include <string>
#include <vector>

namespace {

using namespace gtann_io;

struct Exit {
    int code;
    std::string msg;
};

class Args {
public:
    // value options (long names, aliases "a,b"), switches, ignored value options
    Args(int argc, char** argv, std::initializer_list<const char*> values, std::initializer_list<const char*> switches,
         std::initializer_list<const char*> ignored = {})
    {
        std::map<std::string, std::string> alias;
        auto reg = [&](const char* spec, std::set<std::string>& into) {
            std::string s(spec);
            const size_t c = s.find(',');
            const std::string name = s.substr(0, c);
            into.insert(name);
            alias["--" + name] = name;
            if (c != std::string::npos) alias["-" + s.substr(c + 1)] = name;
        };
        std::set<std::string> vals, sws, ign;
        for (const char* v : values) reg(v, vals);
        for (const char* v : switches) reg(v, sws);
        for (const char* v : ignored) reg(v, ign);
        for (int i = 0; i < argc; ++i) {
            std::string a = argv[i], val;
            bool has_val = false;
            const size_t eq = a.find('=');
            if (a.rfind("--", 0) == 0 && eq != std::string::npos) {
                val = a.substr(eq + 1);
                a = a.substr(0, eq);
                has_val = true;
            }
            auto it = alias.find(a);
            if (it == alias.end()) throw Exit{1, "unknown option " + a};
            const std::string& name = it->second;
            if (sws.count(name)) {
                flags_.insert(name);
                continue;
            }
            if (!has_val) {
                if (i + 1 >= argc) throw Exit{1, "option " + a + " needs a value"};
                val = argv[++i];
            }
            if (!ign.count(name)) kv_[name] = val;
        }
    }
    bool has(const std::string& k) const { return kv_.count(k) > 0; }
    bool flag(const std::string& k) const { return flags_.count(k) > 0; }
    std::string str(const std::string& k) const
    {
        auto it = kv_.find(k);
        if (it == kv_.end()) throw Exit{1, "missing required option --" + k};
        return it->second;
    }
    long long num(const std::string& k, long long def) const { return has(k) ? std::stoll(str(k)) : def; }
    double real(const std::string& k, double def) const { return has(k) ? std::stod(str(k)) : def; }

private:
    std::map<std::string, std::string> kv_;
    std::set<std::string> flags_;
};

struct Lib {
    gt_ctx* ctx = nullptr;
    Lib()
    {
        if (gt_create(0, &ctx) != GT_OK) throw Exit{1, "cannot create a GPU context (gt_create)"};
    }
    ~Lib() { gt_destroy(ctx); }
    void check(int rc, const char* what) const
    {
        if (rc == GT_OK) return;
        const std::string m = std::string(what) + ": " + gt_last_error(ctx);
        throw Exit{rc == GT_ENOMEM ? 2 : 1, m};
    }
};

int dtype_code(Elem e) { return e == Elem::F32 ? GT_DTYPE_F32 : e == Elem::U8 ? GT_DTYPE_U8 : GT_DTYPE_I8; }

double now()
{
    return std::chrono::duration<double>(std::chrono::steady_clock::now().time_since_epoch()).count();
}

void mkdirs(const std::string& path)
{
    std::string cur;
    for (size_t i = 0; i <= path.size(); ++i) {
        if (i == path.size() || path[i] == '/') {
            if (!cur.empty()) mkdir(cur.c_str(), 0755);
        }
        if (i < path.size()) cur.push_back(path[i]);
    }
    struct stat st;
    if (stat(path.c_str(), &st) != 0 || !S_ISDIR(st.st_mode)) throw Exit{1, "cannot create directory " + path};
}

std::string ext_of(const std::string& p)
{
    const size_t dot = p.find_last_of('.');
    const size_t slash = p.find_last_of('/');
    if (dot == std::string::npos || (slash != std::string::npos && dot < slash)) return "";
    return p.substr(dot);
}

std::vector<int64_t> widen(const int32_t* v, size_t n)
{
    return std::vector<int64_t>(v, v + n);
}

// vector_knn.bin -> uint32 table in rank order (src/optimize.cu:89-134)
std::vector<uint32_t> sanitized(const Lib& L, const Table<int32_t>& knn)
{
    std::vector<uint32_t> s(knn.v.size());
    L.check(gt_sanitize(L.ctx, knn.v.data(), knn.N, knn.W, s.data()), "gt_sanitize");
    return s;
}

int cmd_bucket2(int argc, char** argv)
{
    Args a(argc, argv,
           {"input,i", "output,o", "centroid-ratio", "seed", "knn-k", "nprobe", "neighbors-m", "iterations,t",
            "fused-optimize-degree", "kmeans-iters", "balance", "refine-passes", "refine-sample", "order-window",
            "gpu-limit", "kmeans-train-fraction"},
           {"skip-dists", "skip-npy", "out-of-core"},
           {"cpu-limit", "bucket-vec-buffer", "sample-rate", "use-pq", "bucket-mem-mb",
            "gpu-bucket-cache-mb", "pq-bits-start", "pq-bits-min", "search-iters", "cache-mb"});
    const std::string in = a.str("input"), root = a.str("output");
    const int knn_k = static_cast<int>(a.num("knn-k", 32));
    const int np_arg = static_cast<int>(a.num("nprobe", 0));
    const int nprobe = np_arg > 0 ? np_arg : knn_k;
    const int M = static_cast<int>(a.num("neighbors-m", 0));
    const int T = static_cast<int>(a.num("iterations", 1));
    const int K = static_cast<int>(a.num("fused-optimize-degree", 0));
    const int ow_arg = static_cast<int>(a.num("order-window", 0));
    if (M <= 0) throw Exit{1, "--neighbors-m must be > 0 (this build always runs the per-vector kNN)"};
    if (nprobe > 256) throw Exit{1, "nprobe exceeds 256"};
    if (T < 1) throw Exit{1, "iterations must be >= 1"};
    if (knn_k < 1) throw Exit{1, "--knn-k must be >= 1"};
    const double t0 = now();
    Dataset ds = read_dataset(in);
    const double t_read = now() - t0;
    const double ratio = a.real("centroid-ratio", 0.01);
    gt_build_params p;
    gt_build_params_default(&p);
    p.n_buckets = static_cast<int32_t>(std::max<double>(1.0, std::llround(ds.N * ratio)));
    p.nprobe = nprobe;
    p.M = M;
    p.K = K > 0 ? K : std::min(M, 32);
    p.rounds = T;
    p.seed = static_cast<uint64_t>(a.num("seed", 42));
    p.kmeans_iters = static_cast<int32_t>(a.num("kmeans-iters", p.kmeans_iters));
    p.balance = static_cast<float>(a.real("balance", p.balance));
    p.refine_passes = static_cast<int32_t>(a.num("refine-passes", 0));
    p.refine_sample = static_cast<int32_t>(a.num("refine-sample", p.refine_sample));
    if (a.has("kmeans-train-fraction")) {
        p.kmeans_train_fraction = static_cast<float>(a.real("kmeans-train-fraction", 1.0));
        if (!(p.kmeans_train_fraction > 0.f && p.kmeans_train_fraction <= 1.f))
            throw Exit{1, "--kmeans-train-fraction must be in (0, 1]"};
    }
    // --gpu-limit (bytes, 0 = auto): a device budget below the tables runs
    // the build out of core (the running table in host memory, chunked)
    if (a.has("gpu-limit") && a.num("gpu-limit", 0) > 0)
        p.device_budget_mb = static_cast<int32_t>(std::max<int64_t>(1, a.num("gpu-limit", 0) >> 20));
    const int64_t C = std::min<int64_t>(p.n_buckets, ds.N);
    // round-1 centroid self-kNN: knn-k columns for the processing order
    // (centroid_knn.bin), nprobe columns for centroid_pool.bin when given
    // (src/bucket.cu:8976-9001)
    const int ck = std::max(knn_k, np_arg);
    if (ck > C - 1) throw Exit{1, "knn-k / nprobe must be < the number of buckets (" + std::to_string(C) + ")"};
    const std::string dir = root + "/k" + std::to_string(knn_k) + "p" + std::to_string(nprobe) + "m" +
                            std::to_string(M) + "t" + std::to_string(T);
    mkdirs(dir);
    std::printf("Output subdir: %s\n", dir.c_str());
    const size_t nm = static_cast<size_t>(ds.N) * M;
    std::vector<int32_t> ids(nm);
    std::vector<float> dists(nm);
    std::vector<uint32_t> graph(K > 0 ? static_cast<size_t>(ds.N) * K : 0);
    std::vector<int32_t> round1(static_cast<size_t>(ds.N));
    std::vector<uint32_t> cknn(static_cast<size_t>(C) * ck);
    std::vector<int32_t> last_bucket(static_cast<size_t>(ds.N));
    std::vector<int64_t> last_cent(static_cast<size_t>(C));
    gt_build_extras ex{};
    ex.round1_bucket = round1.data();
    ex.centroid_knn = cknn.data();
    ex.centroid_knn_k = ck;
    ex.last_bucket = last_bucket.data();
    ex.last_centroids = last_cent.data();
    gt_build_stats st;
    Lib L;
    L.check(gt_build_graph_ex(L.ctx, ds.data(), ds.N, ds.D, dtype_code(ds.elem), &p, ids.data(), dists.data(),
                              K > 0 ? graph.data() : nullptr, &st, &ex),
            "gt_build_graph_ex");

    // inline reorder of round 1 (src/bucket.cu:9160-9460): buckets in the
    // DiskJoin order of the centroid graph, new ids bucket-contiguous
    const double t1 = now();
    auto columns = [&](int w) {
        std::vector<uint32_t> g(static_cast<size_t>(C) * w);
        for (int64_t c = 0; c < C; ++c)
            std::copy(cknn.begin() + c * ck, cknn.begin() + c * ck + w, g.begin() + c * w);
        return g;
    };
    const std::vector<uint32_t> cgraph = columns(knn_k);
    const int window = ow_arg > 0 ? ow_arg : std::max(4 * knn_k, 16);
    std::vector<int32_t> order(static_cast<size_t>(C));
    L.check(gt_bucket_order(L.ctx, cgraph.data(), C, knn_k, window, order.data()), "gt_bucket_order");
    std::vector<uint32_t> inv(static_cast<size_t>(ds.N)), offsets(static_cast<size_t>(C) + 1);
    L.check(gt_bucket_reorder(L.ctx, round1.data(), ds.N, C, order.data(), nullptr, 0, inv.data(), offsets.data(),
                              nullptr),
            "gt_bucket_reorder");
    std::vector<uint8_t> reordered(ds.bytes.size());
    L.check(gt_permute_rows(L.ctx, ds.data(), ds.N, ds.D, dtype_code(ds.elem), inv.data(), reordered.data()),
            "gt_permute_rows");
    std::vector<int32_t> ids_new(nm);
    L.check(gt_remap_table(L.ctx, ids.data(), ds.N, M, inv.data(), ids_new.data()), "gt_remap_table");
    const double t_reorder = now() - t1;

    const double t2 = now();
    write_dataset(dir + "/data_reordered" + ext_of(in), reordered.data(), ds.N, ds.D, ds.elem);
    write_inverse_perm(dir + "/inverse_perm.bin", inv.data(), ds.N);
    write_bucket_offsets(dir + "/bucket_offsets.bin", offsets.data(), static_cast<int32_t>(C));
    write_bucket_process_order(dir + "/bucket_process_order.bin", order.data(), static_cast<int32_t>(C));
    write_table<uint32_t>(dir + "/centroid_knn.bin", cgraph.data(), C, knn_k);
    if (np_arg > 0) {
        const std::vector<uint32_t> pool = columns(np_arg);
        write_table<uint32_t>(dir + "/centroid_pool.bin", pool.data(), C, np_arg);
    }
    write_table<int32_t>(dir + "/vector_knn.bin", ids_new.data(), ds.N, M);
    if (!a.flag("skip-dists")) {
        std::vector<float> d_new(nm);
        L.check(gt_permute_rows(L.ctx, dists.data(), ds.N, M, GT_DTYPE_F32, inv.data(), d_new.data()),
                "gt_permute_rows");
        write_table<float>(dir + "/vector_dists.bin", d_new.data(), ds.N, M);
    }
    if (!a.flag("skip-npy")) {
        const std::vector<int64_t> w = widen(ids_new.data(), ids_new.size());
        write_npy<int64_t>(dir + "/neighbors.npy", w.data(), ds.N, M);
    }
    if (K > 0) write_table<uint32_t>(dir + "/final_graph.bin", graph.data(), ds.N, K);   // original ids
    {
        // Step 5 (src/bucket.cu:9552-9568): the last round's buckets and
        // centroid rows, in new ids like every later round of the reference
        std::vector<uint32_t> perm(static_cast<size_t>(ds.N));
        for (int64_t n = 0; n < ds.N; ++n) perm[inv[static_cast<size_t>(n)]] = static_cast<uint32_t>(n);
        std::vector<int32_t> bucket_new(static_cast<size_t>(ds.N));
        for (int64_t n = 0; n < ds.N; ++n) bucket_new[static_cast<size_t>(n)] = last_bucket[inv[static_cast<size_t>(n)]];
        write_bucket_files(dir + "/bucket_index.bin", dir + "/bucket_data.bin", bucket_new.data(), ds.N, C);
        std::vector<int64_t> cent_new(static_cast<size_t>(C));
        for (int64_t c = 0; c < C; ++c) cent_new[static_cast<size_t>(c)] = perm[static_cast<size_t>(last_cent[static_cast<size_t>(c)])];
        write_centroid_indices(dir + "/centroid_global_indices.bin", cent_new.data(), C);
    }
    const double t_write = now() - t2;
    std::printf("[bucket2] N=%d D=%d buckets=%lld nprobe=%d M=%d K=%d t=%d order-window=%d\n", ds.N, ds.D,
                static_cast<long long>(C), nprobe, M, K, T, window);
    std::printf("[bucket2] read %.3f s  build %.3f s (bucketing %.3f, knn %.3f, merge %.3f, refine %.3f, prune %.3f, "
                "revmerge %.3f)  reorder %.3f s  write %.3f s\n",
                t_read, st.t_total, st.t_bucketing, st.t_knn, st.t_merge, st.t_refine, st.t_prune, st.t_revmerge,
                t_reorder, t_write);
    return 0;
}

int cmd_optimize(int argc, char** argv)
{
    Args a(argc, argv, {"input,i", "knn-graph,g", "output,o", "output-degree"},
           {"skip-sort", "save-npy", "force-chunked"}, {"gpu-fit-margin"});
    const int K = static_cast<int>(a.num("output-degree", 32));
    if (!a.flag("skip-sort"))
        std::fprintf(stderr, "[optimize] rows are taken in their stored (rank) order, as with --skip-sort\n");
    Table<int32_t> knn = read_table<int32_t>(a.str("knn-graph"));
    Lib L;
    std::vector<uint32_t> s = sanitized(L, knn);
    std::vector<uint32_t> out(static_cast<size_t>(knn.N) * K);
    L.check(gt_optimize(L.ctx, s.data(), knn.N, knn.W, K, out.data()), "gt_optimize");
    write_table<uint32_t>(a.str("output"), out.data(), knn.N, K);
    if (a.flag("save-npy")) {
        std::vector<int64_t> w(out.begin(), out.end());
        write_npy<int64_t>(a.str("output") + ".npy", w.data(), knn.N, K);
    }
    return 0;
}

// src/prune_windowed.cpp: the windowed prune of a bucket2 output directory
// (reordered candidates, bucket_offsets.bin, bucket_process_order.bin,
// centroid_knn.bin or --pool-graph).  The window of processing position p is
// p itself plus the positions of its bucket's centroid-kNN (or pool)
// neighbours, sorted and distinct (src/prune_windowed.cpp:370-385, the
// neighbours as adjacency_from_flat_graph keeps them); --cache-mb is the
// device budget of the chunked prune.  Candidates are ranked as stored (the
// --dists ranking of rows bucket2 wrote sorted).  Without the bucket files
// the whole table is one window: sanitize + full prune, as optimize does.
int cmd_prune_windowed(int argc, char** argv)
{
    Args a(argc, argv,
           {"vector-knn-reordered,k", "dataset,i", "output,o", "output-degree", "bucket-offsets",
            "bucket-process-order", "centroid-knn,c", "cache-mb", "pool-graph"},
           {"save-npy"}, {"order-window", "dists"});
    const int K = static_cast<int>(a.num("output-degree", 32));
    Table<int32_t> knn = read_table<int32_t>(a.str("vector-knn-reordered"));
    if (K > knn.W) throw Exit{1, "--output-degree (" + std::to_string(K) + ") > input degree (" +
                                     std::to_string(knn.W) + ")"};
    Lib L;
    std::vector<uint32_t> out(static_cast<size_t>(knn.N) * K);
    if (a.has("bucket-offsets") && a.has("bucket-process-order") && a.has("centroid-knn")) {
        const std::vector<uint32_t> off = read_bucket_offsets(a.str("bucket-offsets"));
        const int32_t nb = static_cast<int32_t>(off.size()) - 1;
        if (nb < 1 || static_cast<int64_t>(off.back()) != knn.N)
            throw Exit{1, "bucket_offsets does not cover the candidate rows"};
        const std::vector<int32_t> order = read_bucket_process_order(a.str("bucket-process-order"));
        if (static_cast<int32_t>(order.size()) != nb)
            throw Exit{1, "bucket_process_order size (" + std::to_string(order.size()) + ") != n_buckets (" +
                              std::to_string(nb) + ")"};
        std::vector<int32_t> pos_of(static_cast<size_t>(nb), -1);
        for (int32_t p = 0; p < nb; ++p) {
            if (order[static_cast<size_t>(p)] < 0 || order[static_cast<size_t>(p)] >= nb)
                throw Exit{1, "bucket_process_order holds an id out of range"};
            pos_of[static_cast<size_t>(order[static_cast<size_t>(p)])] = p;
        }
        const Table<uint32_t> g = read_table<uint32_t>(a.has("pool-graph") ? a.str("pool-graph") : a.str("centroid-knn"));
        if (g.N != nb) throw Exit{1, "window graph rows (" + std::to_string(g.N) + ") != n_buckets"};
        const int32_t W = g.W + 1;
        std::vector<int32_t> win(static_cast<size_t>(nb) * W, 0), wl(static_cast<size_t>(nb), 0);
        for (int32_t p = 0; p < nb; ++p) {
            const int32_t bkt = order[static_cast<size_t>(p)];
            std::vector<int32_t> w{p};
            for (int32_t k = 0; k < g.W; ++k) {
                const uint32_t nbk = g.v[static_cast<size_t>(bkt) * g.W + k];
                if (static_cast<int64_t>(nbk) != bkt && static_cast<int64_t>(nbk) < nb)
                    w.push_back(pos_of[nbk]);
            }
            std::sort(w.begin(), w.end());
            w.erase(std::unique(w.begin(), w.end()), w.end());
            std::copy(w.begin(), w.end(), win.begin() + static_cast<int64_t>(p) * W);
            wl[static_cast<size_t>(p)] = static_cast<int32_t>(w.size());
        }
        const int64_t budget = static_cast<int64_t>(a.num("cache-mb", 4000)) << 20;
        L.check(gt_prune_windowed(L.ctx, knn.v.data(), knn.N, knn.W, off.data(), nb, win.data(), wl.data(), W, K,
                                  budget, out.data()),
                "gt_prune_windowed");
    } else {
        std::vector<uint32_t> s = sanitized(L, knn);
        L.check(gt_cagra_prune(L.ctx, s.data(), knn.N, knn.W, K, out.data()), "gt_cagra_prune");
    }
    write_table<uint32_t>(a.str("output"), out.data(), knn.N, K);
    return 0;
}

int cmd_optimize_chunked(int argc, char** argv)
{
    Args a(argc, argv, {"forward-graph,g", "output,o", "method,m", "inverse-perm", "final-output", "gpu-budget-mb"},
           {"save-npy"}, {"host-budget-mb", "edge-buffer-mb", "tmp-dir", "bucket-offsets", "rev-degree-cap"});
    if (a.has("method") && a.str("method") != "E") throw Exit{1, "only method E is provided"};
    Table<uint32_t> fwd = read_table<uint32_t>(a.str("forward-graph"));
    Lib L;
    std::vector<uint32_t> out(fwd.v.size());
    // the resident merge when its edge keys and rows fit --gpu-budget-mb, else
    // destination chunks (src/optimize_chunked.cu:1548-2057)
    const int64_t budget = static_cast<int64_t>(a.num("gpu-budget-mb", 8000)) << 20;
    if (static_cast<int64_t>(fwd.v.size()) * 32 <= budget)
        L.check(gt_reverse_merge(L.ctx, fwd.v.data(), fwd.N, fwd.W, out.data()), "gt_reverse_merge");
    else
        L.check(gt_reverse_merge_chunked(L.ctx, fwd.v.data(), fwd.N, fwd.W, budget, out.data()),
                "gt_reverse_merge_chunked");
    write_table<uint32_t>(a.str("output"), out.data(), fwd.N, fwd.W);
    if (a.has("inverse-perm") && a.has("final-output")) {
        std::vector<uint32_t> inv = read_inverse_perm(a.str("inverse-perm"));
        if (static_cast<int64_t>(inv.size()) != fwd.N) throw Exit{1, "inverse permutation length != N"};
        std::vector<uint32_t> fin(out.size());
        L.check(gt_translate(L.ctx, out.data(), inv.data(), fwd.N, fwd.W, fin.data()), "gt_translate");
        write_table<uint32_t>(a.str("final-output"), fin.data(), fwd.N, fwd.W);
    }
    return 0;
}

int cmd_translate(int argc, char** argv)
{
    Args a(argc, argv, {"graph,g", "inverse-perm,p", "output,o"}, {}, {"out-buffer-mb"});
    Table<uint32_t> g = read_table<uint32_t>(a.str("graph"));
    std::vector<uint32_t> inv = read_inverse_perm(a.str("inverse-perm"));
    if (static_cast<int64_t>(inv.size()) != g.N) throw Exit{1, "inverse permutation length != N"};
    Lib L;
    std::vector<uint32_t> out(g.v.size());
    L.check(gt_translate(L.ctx, g.v.data(), inv.data(), g.N, g.W, out.data()), "gt_translate");
    write_table<uint32_t>(a.str("output"), out.data(), g.N, g.W);
    return 0;
}

int cmd_knn(int argc, char** argv)
{
    Args a(argc, argv, {"input,i", "output,o", "k,k"}, {"skip-npy"});
    const int k = static_cast<int>(a.num("k", 32));
    Dataset ds = read_dataset(a.str("input"));
    Lib L;
    const size_t nk = static_cast<size_t>(ds.N) * k;
    std::vector<int32_t> ids(nk);
    std::vector<float> d(nk);
    L.check(gt_knn_exact(L.ctx, ds.data(), ds.N, ds.D, dtype_code(ds.elem), GT_METRIC_L2, nullptr, ds.N, k,
                         ids.data(), d.data()),
            "gt_knn_exact");
    const std::string dir = a.str("output");
    mkdirs(dir);
    write_table<int32_t>(dir + "/vector_knn.bin", ids.data(), ds.N, k);
    write_table<float>(dir + "/vector_dists.bin", d.data(), ds.N, k);
    if (!a.flag("skip-npy")) {
        const std::vector<int64_t> w = widen(ids.data(), ids.size());
        write_npy<int64_t>(dir + "/exact_knn_idx.npy", w.data(), ds.N, k);
        write_npy<float>(dir + "/exact_knn_dist.npy", d.data(), ds.N, k);
    }
    return 0;
}

// Base / query files as bd/search.cpp:227-245 reads them: .u8bin and .i8bin
// bytes as uint8, .ibin as int32 converted to float, anything else float32.
struct SearchData {
    int32_t N = 0, D = 0;
    int dtype = GT_DTYPE_F32;
    std::vector<uint8_t> u8;
    std::vector<float> f32;
    const void* data() const { return dtype == GT_DTYPE_U8 ? static_cast<const void*>(u8.data())
                                                           : static_cast<const void*>(f32.data()); }
    void to_float()
    {
        if (dtype == GT_DTYPE_F32) return;
        f32.assign(u8.begin(), u8.end());
        u8.clear();
        dtype = GT_DTYPE_F32;
    }
};

SearchData read_search_data(const std::string& path)
{
    SearchData s;
    const std::string ext = ext_of(path);
    File f(path, "rb");
    int32_t hdr[2];
    f.read(hdr, sizeof(hdr), "header");
    if (hdr[0] <= 0 || hdr[1] <= 0) throw Exit{1, "bad header (N, D) in " + path};
    s.N = hdr[0];
    s.D = hdr[1];
    const size_t n = static_cast<size_t>(s.N) * s.D;
    if (ext == ".u8bin" || ext == ".i8bin") {
        s.dtype = GT_DTYPE_U8;
        s.u8.resize(n);
        f.read(s.u8.data(), n, "payload");
    } else if (ext == ".ibin") {
        std::vector<int32_t> t(n);
        f.read(t.data(), n * 4, "payload");
        s.f32.assign(t.begin(), t.end());
    } else {
        s.f32.resize(n);
        f.read(s.f32.data(), n * 4, "payload");
    }
    return s;
}

// rows scaled to unit length as bd/search.cpp:280-296 does
void normalize_rows(SearchData& s)
{
    s.to_float();
    for (int64_t i = 0; i < s.N; ++i) {
        float* r = s.f32.data() + i * s.D;
        float norm = 0.f;
        for (int j = 0; j < s.D; ++j) norm += r[j] * r[j];
        norm = std::sqrt(norm + 1e-12f);
        for (int j = 0; j < s.D; ++j) r[j] /= norm;
    }
}

std::vector<uint32_t> read_index(const std::string& path, int64_t N, int32_t& deg)
{
    std::vector<uint32_t> g;
    if (ext_of(path) == ".npy") {
        int64_t rows = 0, cols = 0;
        const std::vector<int64_t> v = read_npy_2d(path, rows, cols);
        if (rows != N) throw Exit{1, "Index N mismatch with base"};
        g.resize(v.size());
        for (size_t i = 0; i < v.size(); ++i)
            g[i] = (v[i] >= 0 && v[i] < N) ? static_cast<uint32_t>(v[i]) : 0xFFFFFFFFu;
        deg = static_cast<int32_t>(cols);
    } else {
        Table<uint32_t> t = read_table<uint32_t>(path);
        if (t.N != N) throw Exit{1, "Index N mismatch with base"};
        g = std::move(t.v);
        deg = t.W;
    }
    return g;
}

// Distinct ids >= 0 of row[0..n), ascending.
template <typename T>
static std::vector<T> distinct_valid(const T* row, int64_t n)
{
    std::vector<T> v;
    v.reserve(static_cast<size_t>(std::max<int64_t>(n, 0)));
    for (int64_t j = 0; j < n; ++j)
        if (row[j] >= 0) v.push_back(row[j]);
    std::sort(v.begin(), v.end());
    v.erase(std::unique(v.begin(), v.end()), v.end());
    return v;
}

// |a ∩ b| of two ascending distinct lists, by one merge pass.
template <typename T>
static int64_t common_count(const std::vector<T>& a, const std::vector<T>& b)
{
    int64_t n = 0;
    for (size_t i = 0, j = 0; i < a.size() && j < b.size();) {
        if (a[i] < b[j]) ++i;
        else if (b[j] < a[i]) ++j;
        else { ++n; ++i; ++j; }
    }
    return n;
}

int cmd_search(int argc, char** argv)
{
    Args a(argc, argv, {"base", "query", "index", "gt", "topk", "ef", "num-entry"}, {"normalize"});
    const int topk = static_cast<int>(a.num("topk", 10));
    int ef = static_cast<int>(a.num("ef", 200));
    const int num_entry = static_cast<int>(a.num("num-entry", 4));
    if (topk < 1 || num_entry < 1 || num_entry > 64) throw Exit{1, "need topk >= 1 and 1 <= num-entry <= 64"};
    std::printf("[eval] Loading data...\n");
    SearchData base = read_search_data(a.str("base"));
    std::printf("  base shape: (%d, %d)\n", base.N, base.D);
    SearchData Q = read_search_data(a.str("query"));
    std::printf("  query shape: (%d, %d)\n", Q.N, Q.D);
    if (Q.D != base.D) throw Exit{1, "Dimension mismatch between base and query"};
    int32_t deg = 0;
    const std::vector<uint32_t> g = read_index(a.str("index"), base.N, deg);
    std::printf("  index shape: (%d, %d)\n", base.N, deg);
    int32_t gt_nq = 0, k_gt = 0;
    const std::vector<int32_t> gt = read_ibin(a.str("gt"), gt_nq, k_gt);
    std::printf("  GT shape: (%d, %d)\n", gt_nq, k_gt);
    if (gt_nq != Q.N) throw Exit{1, "GT nq mismatch with query"};
    if (a.flag("normalize")) {
        std::printf("[eval] L2-normalizing base & queries\n");
        normalize_rows(base);
        normalize_rows(Q);
    }
    if (base.dtype != Q.dtype) {   // one side .u8bin, the other float: search in float
        base.to_float();
        Q.to_float();
    }
    ef = std::max(ef, topk);
    // entry points as bd/search.cpp:51-59 draws them: one generator for all
    // queries, distinct ids in draw order
    std::mt19937 rng(42);
    std::uniform_int_distribution<int> pick(0, base.N - 1);
    std::vector<int32_t> entries(static_cast<size_t>(Q.N) * num_entry, -1);
    for (int32_t i = 0; i < Q.N; ++i) {
        int n = 0;
        for (int e = 0; e < num_entry; ++e) {
            const int s = pick(rng);
            int32_t* row = entries.data() + static_cast<size_t>(i) * num_entry;
            if (std::find(row, row + n, s) == row + n) row[n++] = s;
        }
    }
    std::printf("[eval] start searching ...\n");
    std::fflush(stdout);
    Lib L;
    gt_search_params p;
    gt_search_params_default(&p);
    p.topk = topk;
    p.ef = ef;
    p.num_entry = num_entry;
    std::vector<int32_t> ids(static_cast<size_t>(Q.N) * topk);
    std::vector<float> d(ids.size());
    gt_search_stats st{};
    L.check(gt_search(L.ctx, base.data(), base.N, base.D, base.dtype, g.data(), deg, Q.data(), Q.N, entries.data(),
                      num_entry, &p, ids.data(), d.data(), &st),
            "gt_search");
    // The figures of bd/search.cpp:147-208 (recall_vs_gt): hit GT[:,0] =
    // the first ground-truth id (when valid) is among the predictions; hit
    // any = some prediction is a valid ground-truth id; overlap = distinct
    // valid predictions among the first k that are ground-truth ids, over k,
    // k = min(topk, distinct valid ground-truth ids, k_gt).
    int hit_first = 0, hit_any = 0;
    float total_overlap = 0.f;
    for (int32_t i = 0; i < Q.N; ++i) {
        const int32_t* pr = ids.data() + static_cast<size_t>(i) * topk;
        const int32_t* gr = gt.data() + static_cast<size_t>(i) * k_gt;
        const std::vector<int32_t> gs = distinct_valid(gr, k_gt);
        const std::vector<int32_t> ps = distinct_valid(pr, topk);
        hit_first += gr[0] >= 0 && std::binary_search(ps.begin(), ps.end(), gr[0]);
        hit_any += common_count(ps, gs) > 0;
        const int k = std::min({topk, static_cast<int>(gs.size()), static_cast<int>(k_gt)});
        if (k > 0) total_overlap += common_count(distinct_valid(pr, k), gs) / static_cast<float>(k);
    }
    const float nqf = static_cast<float>(Q.N > 0 ? Q.N : 1);
    std::printf("\n======== Recall vs GT ========\n");
    std::printf("Recall@%d (hit GT[:,0])         : %.6f\n", topk, hit_first / nqf);
    std::printf("Recall@%d (hit any of GT[:,:]) : %.6f\n", topk, hit_any / nqf);
    std::printf("Recall@%d (recall mean overlap): %.6f\n", topk, total_overlap / nqf);
    std::printf("[eval] %d queries in %.3f s on the GPU (%.0f QPS), %.1f expansions per query\n", Q.N, st.t_search,
                Q.N / std::max(st.t_search, 1e-9), st.expansions / static_cast<double>(std::max(Q.N, 1)));
    return 0;
}

int cmd_compare(int argc, char** argv)
{
    Args a(argc, argv, {"index1", "index2", "k-cmp", "k_cmp", "save-csv", "save_csv"}, {});
    int64_t Na = 0, Ma = 0, Nb = 0, Mb = 0;
    const std::vector<int64_t> A = read_npy_2d(a.str("index1"), Na, Ma);
    const std::vector<int64_t> B = read_npy_2d(a.str("index2"), Nb, Mb);
    if (Na != Nb) throw Exit{1, "N mismatch between indices"};
    const long long kc = a.has("k-cmp") ? a.num("k-cmp", -1) : a.num("k_cmp", -1);
    int64_t k = kc > 0 ? kc : std::min(Ma, Mb);
    k = std::min(k, std::min(Ma, Mb));
    if (k <= 0) throw Exit{1, "k_cmp must be > 0"};
    const std::string csv = a.has("save-csv") ? a.str("save-csv") : a.has("save_csv") ? a.str("save_csv") : "";
    std::FILE* fc = nullptr;
    if (!csv.empty()) {
        fc = std::fopen(csv.c_str(), "w");
        if (!fc) throw Exit{1, "cannot write " + csv};
        std::fprintf(fc, "node,intersect_size,deg_A,deg_B,overlap\n");
    }
    int64_t hits_any = 0, set_equal = 0;
    float total = 0.f;
    for (int64_t i = 0; i < Na; ++i) {
        const std::vector<int64_t> SA = distinct_valid(A.data() + static_cast<size_t>(i * Ma), k);
        const std::vector<int64_t> SB = distinct_valid(B.data() + static_cast<size_t>(i * Mb), k);
        const int64_t inter = common_count(SA, SB);
        const float ov = inter / static_cast<float>(k);
        total += ov;
        hits_any += inter >= 1;
        set_equal += static_cast<int64_t>(SA.size()) == k && static_cast<int64_t>(SB.size()) == k && inter == k;
        if (fc) std::fprintf(fc, "%lld,%lld,%zu,%zu,%.6f\n", static_cast<long long>(i), static_cast<long long>(inter),
                             SA.size(), SB.size(), ov);
    }
    if (fc) std::fclose(fc);
    const float n = static_cast<float>(Na > 0 ? Na : 1);
    std::printf("\n======= Index Comparison (set-wise) =======\n");
    std::printf("N=%lld, k=%lld (A:%lld, B:%lld)\n", static_cast<long long>(Na), static_cast<long long>(k),
                static_cast<long long>(Ma), static_cast<long long>(Mb));
    std::printf("MeanOverlap@%lld (|A\u2229B|/k) : %.6f\n", static_cast<long long>(k), total / n);
    std::printf("HitsAny@%lld               : %.6f\n", static_cast<long long>(k), hits_any / n);
    std::printf("SetEqual@%lld              : %.6f\n", static_cast<long long>(k), set_equal / n);
    if (!csv.empty()) std::printf("[compare] per-node stats saved to: %s\n", csv.c_str());
    return 0;
}

void usage()
{
    std::fprintf(stderr,
                 "usage: gtann <bucket2|optimize|prune_windowed|optimize_chunked|translate_ids|knn|search|compare> "
                 "[options]\n");
}

}  // namespace

int main(int argc, char** argv)
{
    if (argc < 2) {
        usage();
        return 1;
    }
    const std::string cmd = argv[1];
    try {
        if (cmd == "bucket2") return cmd_bucket2(argc - 2, argv + 2);
        if (cmd == "optimize") return cmd_optimize(argc - 2, argv + 2);
        if (cmd == "prune_windowed") return cmd_prune_windowed(argc - 2, argv + 2);
        if (cmd == "optimize_chunked") return cmd_optimize_chunked(argc - 2, argv + 2);
        if (cmd == "translate_ids") return cmd_translate(argc - 2, argv + 2);
        if (cmd == "knn") return cmd_knn(argc - 2, argv + 2);
        if (cmd == "search") return cmd_search(argc - 2, argv + 2);
        if (cmd == "compare") return cmd_compare(argc - 2, argv + 2);
        usage();
        return 1;
    } catch (const Exit& e) {
        std::fprintf(stderr, "FATAL: %s\n", e.msg.c_str());
        return e.code;
    } catch (const std::exception& e) {
        std::fprintf(stderr, "FATAL: %s\n", e.what());
        return 1;
    }
}
