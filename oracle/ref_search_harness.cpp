// Test-time harness over the reference's own C++ graph search
// (bd/search.cpp:33-137, graph_search_single), compiled where it lies: the
// Makefile passes the source path as REF_SEARCH_CPP and renames its main().
// Exposes one C entry point that runs the reference's per-query search with
// a single std::mt19937(seed) shared across queries, as its
// search_graph_recall does (bd/search.cpp:305-320), and also reports the
// entry points each query drew (replaying the same distribution on a copy of
// the generator), so the oracle can be run from the same entries.
#include REF_SEARCH_CPP

extern "C" int ref_graph_search(const float* X, int32_t N, int32_t D, const int64_t* graph, int32_t M,
                                const float* Q, int32_t nq, int32_t topk, int32_t ef, int32_t num_entry,
                                uint32_t seed, int64_t* out_ids, float* out_d, int32_t* entries)
{
    try {
        std::vector<float> base(X, X + static_cast<size_t>(N) * D);
        std::vector<int64_t> nb(graph, graph + static_cast<size_t>(N) * M);
        std::mt19937 rng(seed);
        ef = std::max(ef, topk);
        for (int32_t i = 0; i < nq; ++i) {
            std::mt19937 replay = rng;
            std::uniform_int_distribution<int> pick(0, N - 1);
            std::vector<int> drawn;
            for (int e = 0; e < num_entry; ++e) {
                const int s = pick(replay);
                if (std::find(drawn.begin(), drawn.end(), s) == drawn.end()) drawn.push_back(s);
            }
            for (int e = 0; e < num_entry; ++e)
                entries[static_cast<size_t>(i) * num_entry + e] = e < static_cast<int>(drawn.size()) ? drawn[e] : -1;
            SearchResult r = graph_search_single(Q + static_cast<size_t>(i) * D, base, nb, N, M, D, topk, ef, rng,
                                                 num_entry);
            for (int32_t j = 0; j < topk; ++j) {
                out_ids[static_cast<size_t>(i) * topk + j] = j < static_cast<int32_t>(r.indices.size()) ? r.indices[j] : -1;
                out_d[static_cast<size_t>(i) * topk + j] =
                    j < static_cast<int32_t>(r.distances.size()) ? r.distances[j] : INFINITY;
            }
        }
        return 0;
    } catch (...) {
        return -1;
    }
}
