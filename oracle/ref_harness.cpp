// ref_harness.cpp -- C entry points over the reference's own CUDA-free
// headers, compiled in place from /root/reference by oracle/Makefile into
// oracle/_ref/libgtann_ref.so.  Test infrastructure only: it lets the tests
// check the CPU restatement (gt_oracle.c) and write golden fixtures against
// the reference implementation itself.  Nothing here is shipped.
//
// Wrapped reference functions:
//   prune_windowed::compute_detour_counts / select_pruned_row
//       (src/prune_windowed_core.hpp:189-263), full window via WindowLookup
//       (src/prune_windowed_core.hpp:50-75), rows taken in the given order,
//       and with a BucketWindow per processing position
//       (src/prune_windowed_core.hpp:77-124) for the windowed prune;
//   edge_chunk::build_rank_ordered_csr + merge_rank_ordered_into_row
//       (src/edge_chunk_accumulator.hpp:235-284, 471-494), fed the reverse
//       edges {dst = fwd[i][k], src = i, rank = k} of
//       src/optimize_chunked.cu:372-407;
//   translate_ids::translate_graph_to_original_order
//       (src/translate_graph_ids.hpp:75), through temporary files;
//   graph_io::write_graph / write_vector_knn / write_vector_bin /
//       read_forward_graph / read_vector_knn (src/graph_io.hpp) and
//       load::read_fbin_f32 / read_u8bin_to_f32 (src/load.hpp:67-117): the
//       on-disk formats, for byte-level checks of this build's writers;
//   bucket_order::compute_bucket_processing_order over
//       adjacency_from_flat_graph (src/bucket_order.hpp:161-262), and
//       graph_io::write/read_bucket_offsets, write/read_bucket_process_order
//       (src/graph_io.hpp:178-244).
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <filesystem>
#include <stdexcept>
#include <string>
#include <vector>
#include <unistd.h>

#include "prune_windowed_core.hpp"
#include "edge_chunk_accumulator.hpp"
#include "graph_io.hpp"
#include "translate_graph_ids.hpp"
#include "load.hpp"
#include "bucket_order.hpp"

extern "C" {

// 0 = ok, -4 = fewer than K valid candidates in some row, -1 = other error
int ref_cagra_prune(const int32_t* G, int64_t N, int32_t M, int32_t K, uint32_t* out)
{
    try {
        prune_windowed::WindowLookup w;
        w.reserve(static_cast<size_t>(N));
        static const float dummy = 0.f;
        for (int64_t i = 0; i < N; ++i)
            w.add(static_cast<uint32_t>(i), G + i * M, &dummy);
        std::vector<uint32_t> detour;
        for (int64_t a = 0; a < N; ++a) {
            prune_windowed::compute_detour_counts(G + a * M, M, w, detour);
            prune_windowed::select_pruned_row(G + a * M, M, detour, K, out + a * K);
        }
        return 0;
    } catch (const std::runtime_error& e) {
        return std::string(e.what()).find("fewer than output_degree") != std::string::npos ? -4 : -1;
    } catch (...) {
        return -1;
    }
}

// The windowed prune as src/prune_windowed.cpp's batched path runs it: per
// processing position p a BucketWindow (src/prune_windowed_core.hpp:77-124)
// holding the buckets win[p*W .. p*W + win_len[p]), then
// compute_detour_counts + select_pruned_row on each row of p's bucket in the
// given order (rows already ranked, as the --dists ranking leaves them).
int ref_prune_windowed(const int32_t* G, int64_t N, int32_t M, const uint32_t* off, int32_t nb, const int32_t* win,
                       const int32_t* win_len, int32_t W, int32_t K, uint32_t* out)
{
    try {
        prune_windowed::BucketWindow bw(off, nb);
        static const float dummy = 0.f;
        std::vector<uint32_t> detour;
        for (int32_t p = 0; p < nb; ++p) {
            bw.clear();
            for (int32_t i = 0; i < win_len[p]; ++i) {
                const int32_t q = win[static_cast<int64_t>(p) * W + i];
                bw.add_bucket(q, G + static_cast<int64_t>(off[q]) * M, M, &dummy, 0);
            }
            for (int64_t a = off[p]; a < static_cast<int64_t>(off[p + 1]); ++a) {
                prune_windowed::compute_detour_counts(G + a * M, M, bw, detour);
                prune_windowed::select_pruned_row(G + a * M, M, detour, K, out + a * K);
            }
        }
        return 0;
    } catch (const std::runtime_error& e) {
        return std::string(e.what()).find("fewer than output_degree") != std::string::npos ? -4 : -1;
    } catch (...) {
        return -1;
    }
}

// The reference CPU prune as its CLI runs it (src/prune_windowed.cpp:97):
// rows in parallel over OpenMP threads, one detour buffer per thread; the
// timed CPU baseline of bench.py.  Same output as ref_cagra_prune.
int ref_cagra_prune_omp(const int32_t* G, int64_t N, int32_t M, int32_t K, uint32_t* out)
{
    try {
        prune_windowed::WindowLookup w;
        w.reserve(static_cast<size_t>(N));
        static const float dummy = 0.f;
        for (int64_t i = 0; i < N; ++i)
            w.add(static_cast<uint32_t>(i), G + i * M, &dummy);
        int64_t n_fail = 0;
        #pragma omp parallel reduction(+:n_fail)
        {
            std::vector<uint32_t> detour;
            #pragma omp for schedule(dynamic, 256)
            for (int64_t a = 0; a < N; ++a) {
                try {
                    prune_windowed::compute_detour_counts(G + a * M, M, w, detour);
                    prune_windowed::select_pruned_row(G + a * M, M, detour, K, out + a * K);
                } catch (...) {
                    ++n_fail;
                }
            }
        }
        return n_fail ? -4 : 0;
    } catch (...) {
        return -1;
    }
}

// The reference's rank-ordered reverse merge with its own OpenMP CSR build
// (src/edge_chunk_accumulator.hpp:235-284) and the rows merged in parallel.
int ref_reverse_merge_omp(const uint32_t* fwd, int64_t N, int32_t K, uint32_t* out)
{
    try {
        std::vector<edge_chunk::EdgeRecord> edges(static_cast<size_t>(N) * K);
        #pragma omp parallel for schedule(static)
        for (int64_t i = 0; i < N; ++i)
            for (int32_t k = 0; k < K; ++k)
                edges[static_cast<size_t>(i * K + k)] =
                    edge_chunk::EdgeRecord{fwd[i * K + k], static_cast<uint32_t>(i), static_cast<uint16_t>(k)};
        auto csr = edge_chunk::build_rank_ordered_csr(edges, 0, static_cast<uint32_t>(N));
        #pragma omp parallel for schedule(dynamic, 1024)
        for (int64_t j = 0; j < N; ++j) {
            uint32_t* row = out + j * K;
            for (int32_t k = 0; k < K; ++k) row[k] = fwd[j * K + k];
            const uint32_t lo = csr.row_offsets[static_cast<size_t>(j)];
            const uint32_t hi = csr.row_offsets[static_cast<size_t>(j) + 1];
            edge_chunk::merge_rank_ordered_into_row(row, csr.src.data() + lo, hi - lo, static_cast<uint32_t>(K));
        }
        return 0;
    } catch (...) {
        return -1;
    }
}

int ref_detour_counts(const int32_t* G, int64_t N, int32_t M, int64_t a, uint32_t* counts)
{
    try {
        prune_windowed::WindowLookup w;
        static const float dummy = 0.f;
        for (int64_t i = 0; i < N; ++i)
            w.add(static_cast<uint32_t>(i), G + i * M, &dummy);
        std::vector<uint32_t> detour;
        prune_windowed::compute_detour_counts(G + a * M, M, w, detour);
        for (int32_t k = 0; k < M; ++k) counts[k] = detour[static_cast<size_t>(k)];
        return 0;
    } catch (...) {
        return -1;
    }
}

int ref_reverse_merge(const uint32_t* fwd, int64_t N, int32_t K, uint32_t* out)
{
    try {
        std::vector<edge_chunk::EdgeRecord> edges;
        edges.reserve(static_cast<size_t>(N) * K);
        for (int64_t i = 0; i < N; ++i)
            for (int32_t k = 0; k < K; ++k)
                edges.push_back(edge_chunk::EdgeRecord{fwd[i * K + k], static_cast<uint32_t>(i),
                                                       static_cast<uint16_t>(k)});
        auto csr = edge_chunk::build_rank_ordered_csr(edges, 0, static_cast<uint32_t>(N));
        for (int64_t j = 0; j < N; ++j) {
            uint32_t* row = out + j * K;
            for (int32_t k = 0; k < K; ++k) row[k] = fwd[j * K + k];
            const uint32_t lo = csr.row_offsets[static_cast<size_t>(j)];
            const uint32_t hi = csr.row_offsets[static_cast<size_t>(j) + 1];
            edge_chunk::merge_rank_ordered_into_row(row, csr.src.data() + lo, hi - lo,
                                                    static_cast<uint32_t>(K));
        }
        return 0;
    } catch (...) {
        return -1;
    }
}

int ref_translate(const uint32_t* g, const uint32_t* inv, int64_t N, int32_t K, uint32_t* out)
{
    try {
        char tmpl[] = "/tmp/gtann_ref_XXXXXX";
        char* dir = mkdtemp(tmpl);
        if (!dir) return -1;
        const std::string d(dir);
        graph_io::write_graph(d + "/g.bin", g, N, K);
        {
            FILE* f = std::fopen((d + "/inv.bin").c_str(), "wb");
            if (!f) return -1;
            std::fwrite(inv, sizeof(uint32_t), static_cast<size_t>(N), f);
            std::fclose(f);
        }
        translate_ids::translate_graph_to_original_order(d + "/g.bin", d + "/inv.bin", d + "/o.bin");
        std::vector<uint32_t> res;
        int64_t n2 = 0;
        int32_t k2 = 0;
        graph_io::read_forward_graph(d + "/o.bin", res, n2, k2);
        std::filesystem::remove_all(d);
        if (n2 != N || k2 != K) return -1;
        for (size_t i = 0; i < res.size(); ++i) out[i] = res[i];
        return 0;
    } catch (...) {
        return -1;
    }
}

int ref_bucket_order(const uint32_t* g, int64_t B, int32_t K, int32_t window, int32_t* order)
{
    try {
        const std::vector<int32_t> o = bucket_order::compute_bucket_processing_order(
            bucket_order::adjacency_from_flat_graph(g, B, K), window);
        std::copy(o.begin(), o.end(), order);
        return 0;
    } catch (...) {
        return -1;
    }
}

int ref_write_bucket_offsets(const char* path, const uint32_t* off, int64_t n_plus_1)
{
    try {
        graph_io::write_bucket_offsets(path, std::vector<uint32_t>(off, off + n_plus_1));
        return 0;
    } catch (...) {
        return -1;
    }
}

int ref_write_bucket_process_order(const char* path, const int32_t* order, int64_t n)
{
    try {
        graph_io::write_bucket_process_order(path, std::vector<int32_t>(order, order + n));
        return 0;
    } catch (...) {
        return -1;
    }
}

// readers: the count is returned through n (entries written to out, capacity cap)
int ref_read_bucket_offsets(const char* path, uint32_t* out, int64_t cap, int64_t* n)
{
    try {
        const std::vector<uint32_t> v = graph_io::read_bucket_offsets(path);
        if (static_cast<int64_t>(v.size()) > cap) return -2;
        std::copy(v.begin(), v.end(), out);
        *n = static_cast<int64_t>(v.size());
        return 0;
    } catch (...) {
        return -1;
    }
}

int ref_read_bucket_process_order(const char* path, int32_t* out, int64_t cap, int64_t* n)
{
    try {
        const std::vector<int32_t> v = graph_io::read_bucket_process_order(path);
        if (static_cast<int64_t>(v.size()) > cap) return -2;
        std::copy(v.begin(), v.end(), out);
        *n = static_cast<int64_t>(v.size());
        return 0;
    } catch (...) {
        return -1;
    }
}

int ref_write_graph(const char* path, const uint32_t* g, int64_t N, int32_t K)
{
    try {
        graph_io::write_graph(path, g, N, K);
        return 0;
    } catch (...) {
        return -1;
    }
}

int ref_write_vector_knn(const char* path, const int32_t* g, int64_t N, int32_t M)
{
    try {
        graph_io::write_vector_knn(path, std::vector<int32_t>(g, g + N * M), N, M);
        return 0;
    } catch (...) {
        return -1;
    }
}

int ref_write_u32_vector(const char* path, const uint32_t* v, int64_t n)
{
    try {
        graph_io::write_vector_bin(path, std::vector<uint32_t>(v, v + n));
        return 0;
    } catch (...) {
        return -1;
    }
}

// reads a graph file into out (capacity cap entries); N, K returned
int ref_read_graph(const char* path, uint32_t* out, int64_t cap, int64_t* N, int32_t* K)
{
    try {
        std::vector<uint32_t> g;
        graph_io::read_forward_graph(path, g, *N, *K);
        if (static_cast<int64_t>(g.size()) > cap) return -1;
        for (size_t i = 0; i < g.size(); ++i) out[i] = g[i];
        return 0;
    } catch (...) {
        return -1;
    }
}

int ref_read_vector_knn(const char* path, int32_t* out, int64_t cap, int64_t* N, int32_t* M)
{
    try {
        graph_io::VectorKnn vk = graph_io::read_vector_knn(path);
        if (static_cast<int64_t>(vk.graph.size()) > cap) return -1;
        *N = vk.N;
        *M = vk.M;
        for (size_t i = 0; i < vk.graph.size(); ++i) out[i] = vk.graph[i];
        return 0;
    } catch (...) {
        return -1;
    }
}

// dataset reader of the C++ pipeline: .fbin/.bin as float, .u8bin/.i8bin
// converted by extension (.i8bin signed)
int ref_read_dataset(const char* path, float* out, int64_t cap, int32_t* N, int32_t* D)
{
    try {
        std::vector<float> v;
        const std::string p(path);
        if (p.size() >= 5 && (p.compare(p.size() - 5, 5, ".fbin") == 0 || p.compare(p.size() - 4, 4, ".bin") == 0))
            load::read_fbin_f32(p, v, *N, *D);
        else
            load::read_u8bin_to_f32(p, v, *N, *D);
        if (static_cast<int64_t>(v.size()) > cap) return -1;
        for (size_t i = 0; i < v.size(); ++i) out[i] = v[i];
        return 0;
    } catch (...) {
        return -1;
    }
}

}  // extern "C"
