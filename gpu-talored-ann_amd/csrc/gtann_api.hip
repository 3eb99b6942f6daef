// gtann_api.hip -- host orchestration and the C ABI of include/gtann.h.
//
// Host C++ owns the control flow (bucketing decisions, work lists, error
// handling); every data-parallel stage is one of the hand-written kernels of
// knn_kernels.hip / graph_kernels.hip / refine_kernel.hip on the context's
// stream.
#include "gtann_common.hpp"

#include <algorithm>
#include <atomic>
#include <chrono>
#include <climits>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <memory>
#include <condition_variable>
#include <functional>
#include <future>
#include <mutex>
#include <numeric>
#include <thread>
#include <unordered_set>
#include <vector>

namespace gtann {
// knn_kernels.hip
void launch_knn_fused(const KnnArgs& a, hipStream_t stream);
// knn_collect.hip
bool knn_collect_supported(const KnnArgs& a);
void launch_knn_collect_select(const KnnArgs& a, int64_t rows, hipStream_t stream);
void launch_merge_partials(const int32_t* pids, const float* pd, int64_t nq, int splits, int M, int32_t* out_ids,
                           float* out_d, hipStream_t stream);
bool resident_supported(const KnnArgs& a, int64_t np);
void launch_knn_resident(const KnnArgs& a, int64_t nq, int64_t np, hipStream_t stream);
// screen_kernels.hip
bool screen_supported(int Dp, int64_t max_pool);
void launch_screen_prepare(const float* X, const float* nrm, int64_t N, int Dp, unsigned int* sq, uint16_t* Xh,
                           hipStream_t s);
void launch_screen(const WorkItem* items, int n_items, const int32_t* pairs, int n_pairs, const int64_t* ubase,
                   const int32_t* q_rows,
                   const int32_t* p_rows, const uint16_t* Xh, const float* nrm, const unsigned int* sq, int Dp,
                   int metric, const float* seed_d, int seed_ld, int M, int wtiles, float* tq, int32_t* union_rows,
                   WorkItem* items_out, unsigned long long* pairs_done, hipStream_t s);
// graph_kernels.hip
void launch_pad_convert(const void* src, int dtype, float* dst, int64_t N, int D, int Dp, hipStream_t s);
void launch_row_norms(const float* X, int64_t N, int Dp, float* norms, hipStream_t s);
void launch_pad_i8(const void* src, int dtype, int8_t* dst, int64_t N, int D, int Dp, hipStream_t s);
void launch_prepare_int(const void* src, int dtype, int64_t N, int D, int Dp, float* xf, float* nf, int8_t* x8,
                        float* n8, hipStream_t s);
void launch_row_norms_i8(const int8_t* X, int64_t N, int Dp, float* norms, hipStream_t s);
void launch_quantize_i8(const float* src, int64_t N, int D, int Dp, int shift, int8_t* dst, hipStream_t s);
void launch_round_to_int(const float* src, int64_t N, int D, int Dp, int shift, float* dst, hipStream_t s);
void launch_row_norms_range(const float* X, int64_t N, int Dp, float* norms, int* part, int* out, hipStream_t s);
void launch_quantize_norms_i8(const float* src, int64_t N, int D, int Dp, int shift, int8_t* dst, float* norms,
                              hipStream_t s);
void launch_segment_sort(const int32_t* members, const int32_t* key, const int64_t* off, int64_t nseg, int min_n,
                         const int32_t* remap, const int64_t* remap_base, int32_t* out, hipStream_t s);
void launch_sub_chain(const int32_t* nn, int K, const int64_t* base, const int32_t* count, int64_t nseg, int32_t* pos,
                      hipStream_t s);
void launch_copy_ranges(const void* tasks, int64_t ntasks, const int32_t* members, int32_t* pool, hipStream_t s);
void launch_negate(float* d, int64_t n, hipStream_t s);
void launch_graph_search(const SearchArgs& a, int64_t grid, hipStream_t s);
void launch_invert_perm(const uint32_t* inv, int64_t N, uint32_t* perm, uint32_t* hits, int* err, hipStream_t s);
void launch_permute_rows(const void* in, const uint32_t* inv, int64_t N, int64_t row_bytes, void* out, hipStream_t s);
void launch_remap_table(const int32_t* ids, const uint32_t* inv, const uint32_t* perm, int64_t N, int M, int32_t* out,
                        hipStream_t s);
size_t search_lds_bytes(int CC, int efr, int Dp, int H);
void launch_sanitize(const int32_t* in, int64_t N, int M, uint32_t* out, hipStream_t s);
void launch_init_flags(unsigned long long* bad_row, int* err, hipStream_t s);
void launch_cagra_prune(const int32_t* G, int64_t N, int M, int K, uint32_t* out, unsigned long long* bad_row,
                        hipStream_t s, const int32_t* order = nullptr, bool flat_rows = false);
void launch_rev_count(const uint32_t* fwd, int64_t N, int K, uint32_t* deg, uint32_t* slot, int* err, hipStream_t s);
void launch_exclusive_scan(const uint32_t* in, int64_t n, uint32_t* out, uint32_t* sums, hipStream_t s);
void launch_chunk_bounds(const int8_t* X8, int Dp, const int32_t* pool, const int32_t* cnt, int64_t nch, int8_t* c8,
                         float* cn, float* cr, hipStream_t s);
void launch_kmpar_init(uint8_t* flag, float* mind, int64_t S, int64_t first, hipStream_t s);
void launch_kmpar_psi(const float* mind, int64_t S, int64_t target, float* psi, hipStream_t s);
void launch_kmpar_sample(const float* mind, uint8_t* flag, uint32_t* sel, int64_t S, const float* psi, float lk,
                         uint64_t seed, hipStream_t s);
void launch_kmpar_compact(const uint32_t* sel, const uint32_t* pos, const int32_t* rows, int64_t S, int32_t* out,
                          hipStream_t s);
void launch_kmpar_min(float* mind, const float* dnew, int64_t S, hipStream_t s);
void launch_gather_rows_f32(const float* X, int Dp, const int32_t* ids, int64_t n, float* out, hipStream_t s);
void launch_rev_scatter(const uint32_t* fwd, int64_t N, int K, const uint32_t* off, const uint32_t* slot,
                        unsigned long long* keys, hipStream_t s);
int rev_bin_shift(int64_t N);
int rev_bin_blocks(int64_t E);
void launch_rev_binned(const uint32_t* fwd, int64_t N, int K, uint32_t* hist, uint32_t* offs, uint32_t* sums,
                       unsigned long long* part, unsigned long long* grouped, uint32_t* out, int* err, hipStream_t s);
bool rv_plan(int64_t N, int K, RvPlan& p);
bool rv_plan2(int64_t N, int K, RvPlan& p);
RvSizes rv_sizes(int64_t N, int K, const RvPlan& p);
void launch_rv(const uint32_t* fwd, int64_t N, int K, const RvPlan& p, const RvBufs& bf, uint32_t* out, int* err,
               uint32_t* slow_rows, uint32_t* slow_count, uint32_t* big_bins, hipStream_t s);
void launch_rev_merge(const uint32_t* fwd, int64_t N, int K, const uint32_t* off, const unsigned long long* keys,
                      uint32_t* out, hipStream_t s);
void launch_occlusion_prune(const float* X, int64_t N, int Dp, const int32_t* nb, int M, int max_deg, int32_t* out,
                            hipStream_t s);
void launch_rin_worst(const float* d, int64_t N, int M, float* worst, hipStream_t s);
void launch_rin_count(const int32_t* ids, const float* d, int64_t N, int M, const float* worst, uint32_t* cnt,
                      uint32_t* slot, int* err, hipStream_t s);
void launch_rin_scatter(const int32_t* ids, const float* d, int64_t N, int M, const uint32_t* off,
                        const uint32_t* slot, unsigned long long* keys, hipStream_t s);
void launch_rin_merge(int32_t* ids, float* d, int64_t N, int M, const uint32_t* off, const unsigned long long* keys,
                      hipStream_t s);
void launch_merge_rounds(const int32_t* ri, const float* rd, const int32_t* ni, const float* nd, int64_t N, int M,
                         int32_t* oi, float* od, hipStream_t s);
void launch_translate(const uint32_t* g, const uint32_t* inv, int64_t N, int K, uint32_t* out, uint32_t* hits,
                      int* err, hipStream_t s);
void launch_cagra_prune_mapped(const int32_t* G, int64_t N, int M, int K, uint32_t* out, unsigned long long* bad_row,
                               const PruneMap& map, int rows_mode, hipStream_t s);
// ooc_kernels.hip
void launch_set_cidx(const int32_t* ids, int64_t n, int32_t* cidx, hipStream_t s);
void launch_route(const uint32_t* fwd, int64_t nrows, int K, int64_t N, int64_t R, int nchunks, int64_t s0,
                  uint32_t* counts, uint32_t* cursor, unsigned long long* recs, int* err, bool place, hipStream_t s);
void launch_rec_group(const unsigned long long* recs, int64_t n, uint32_t* deg, uint32_t* slot, const uint32_t* off,
                      unsigned long long* keys, bool scatter, hipStream_t s);
// refine_kernel.hip
void launch_refine_2hop(const float* X, const float* norms, int64_t N, int Dp, int metric, const int32_t* order,
                        const int32_t* in_ids, const float* in_d, int M, int S, int32_t* out_ids, float* out_d,
                        hipStream_t s);
void launch_centroid_sums(const float* X, int Dp, const int32_t* members, const int64_t* offsets, int64_t C,
                          float* centroids, hipStream_t s);
int csr_blocks(int64_t S);
void launch_sample_csr(const int32_t* key, const int32_t* val, int64_t S, int C, uint32_t* hist, uint32_t* offs,
                       uint32_t* sums, int32_t* members, int64_t* off, hipStream_t s);
void launch_gather_i32(const int32_t* src, const int32_t* idx, int64_t n, int32_t* out, hipStream_t s);
void launch_pack_u16(const uint32_t* in, int64_t n, uint16_t* out, hipStream_t s);
void launch_bucket_csr(const uint32_t* top2, const int32_t* bucket, int64_t N, int C, int32_t* key2, int32_t* by_key,
                       int32_t* bkt, uint32_t* hist, uint32_t* offs, uint32_t* sums, int32_t* members, int64_t* off,
                       hipStream_t s);

struct CopyTaskH { int64_t src; int64_t dst; int64_t n; };

// ---------------------------------------------------------------- device memory

struct DevBuf {
    void* p = nullptr;
    size_t cap = 0;
    DevBuf() = default;
    DevBuf(const DevBuf&) = delete;
    DevBuf& operator=(const DevBuf&) = delete;
    ~DevBuf() { if (p) (void)hipFree(p); }
    void* ensure(size_t bytes) {
        if (bytes <= cap) return p;
        if (p) GT_HIP(hipFree(p));
        p = nullptr;
        cap = 0;
        GT_HIP(hipMalloc(&p, std::max<size_t>(bytes, 256)));
        cap = std::max<size_t>(bytes, 256);
        return p;
    }
    template <typename T> T* as(size_t n) { return static_cast<T*>(ensure(n * sizeof(T))); }
};

// Pinned host staging (hipHostMalloc), grown on demand and reused.
struct HostBuf {
    void* p = nullptr;
    size_t cap = 0;
    HostBuf() = default;
    HostBuf(const HostBuf&) = delete;
    HostBuf& operator=(const HostBuf&) = delete;
    ~HostBuf() { release(); }
    void release()
    {
        if (p) (void)hipHostFree(p);
        p = nullptr;
        cap = 0;
    }
    void* ensure(size_t bytes)
    {
        if (bytes <= cap) return p;
        release();
        GT_HIP(hipHostMalloc(&p, std::max<size_t>(bytes, 4096), hipHostMallocDefault));
        cap = std::max<size_t>(bytes, 4096);
        return p;
    }
    template <typename T> T* as(size_t n) { return static_cast<T*>(ensure(n * sizeof(T))); }
};

static bool is_device_ptr(const void* p)
{
    if (!p) return false;
    hipPointerAttribute_t attr;
    if (hipPointerGetAttributes(&attr, p) != hipSuccess) {
        (void)hipGetLastError();
        return false;
    }
    return attr.type == hipMemoryTypeDevice;
}

struct Timer {
    std::chrono::steady_clock::time_point t0 = std::chrono::steady_clock::now();
    double sec() const { return std::chrono::duration<double>(std::chrono::steady_clock::now() - t0).count(); }
};

// Stage tracing: with GTANN_TRACE=1 in the environment every mark()
// synchronises the stream and prints the wall time since the previous mark
// to stderr.  Off (the default) it costs nothing and adds no synchronisation.
struct Trace {
    bool on = false;
    Timer t;
    Trace()
    {
        const char* e = std::getenv("GTANN_TRACE");
        on = e && e[0] && e[0] != '0';
    }
    void mark(hipStream_t s, const char* what)
    {
        if (!on) return;
        (void)hipStreamSynchronize(s);
        std::fprintf(stderr, "[gtann] %-28s %9.3f ms\n", what, t.sec() * 1e3);
        t = Timer();
    }
};

}  // namespace gtann

namespace gtann {

// Allocator over pinned host memory (hipHostMalloc): a vector whose upload
// is a DMA transfer the host does not wait for.
template <class T> struct PinnedAlloc {
    using value_type = T;
    PinnedAlloc() = default;
    template <class U> PinnedAlloc(const PinnedAlloc<U>&) {}
    T* allocate(size_t n) {
        void* p = nullptr;
        if (hipHostMalloc(&p, n * sizeof(T), hipHostMallocDefault) != hipSuccess) throw std::bad_alloc();
        return static_cast<T*>(p);
    }
    void deallocate(T* p, size_t) { (void)hipHostFree(p); }
    template <class U> bool operator==(const PinnedAlloc<U>&) const { return true; }
    template <class U> bool operator!=(const PinnedAlloc<U>&) const { return false; }
};
using PinnedI32 = std::vector<int32_t, PinnedAlloc<int32_t>>;

}  // namespace gtann

struct gt_ctx {
    int device = 0;
    hipStream_t stream = nullptr;
    std::string err;
    // named workspaces, grow-only (one slot per role, see gtann::Ws)
    gtann::DevBuf ws[112];
    gtann::HostBuf pinned[2];   // top-2 assignment downloads of two consecutive rounds
    gtann::HostBuf pin_lloyd;   // Lloyd steps: nearest centroids down, CSR up
    gtann::HostBuf pin_bucket[2];   // two-choice buckets of two consecutive rounds (uploaded for the device CSR)
    // host scratch of the bucketing, reused across calls (no page faults on
    // fresh N-sized allocations every round)
    std::vector<int32_t> h_bucket_of, h_key2, h_by_key, h_bkt;
    gtann::PinnedI32 h_members[2];
    hipEvent_t members_up[2] = {nullptr, nullptr};   // after the last upload of h_members[i]
    int64_t knn_launches = 0;   // bucketed-round launches of the current build
    double knn_pairs_done = 0;  // (query, pool row) pairs the collect kernels computed (chunk pruning skips the rest)
    uint64_t members_gen = 0;   // bucketing whose members W_MEMBERS holds (0: none)
    uint64_t data_gen = 0;      // bumped whenever W_X / W_NORMS are (re)written
    uint64_t screen_gen = 0;    // data_gen whose fp16 copy and scale W_XH / W_SQ hold (0: none)
    const float* screen_src = nullptr;
    hipEvent_t ev0 = nullptr, ev1 = nullptr;
    void* scratch = nullptr;    // this device's fixed scratch array (gt_optimize_noalloc), or null
    std::string scratch_err;    // why it is null
    gt_debug_opts dbg{};        // path selection (gt_set_debug)
};

namespace gtann {

enum Ws {
    W_X, W_XRAW, W_NORMS, W_C, W_CRAW, W_CNORMS, W_IDS, W_D, W_IDS2, W_D2, W_IDS3, W_D3, W_ITEMS, W_QROWS, W_PROWS,
    W_MEMBERS, W_TASKS, W_POOL, W_PART_I, W_PART_D, W_G1, W_G2, W_G3, W_DEG, W_OFF, W_CUR, W_KEYS, W_SUMS, W_FLAG,
    W_TMP, W_OUT, W_IN, W_PROBE_I, W_PROBE_D, W_WORST, W_X8, W_NORMS8, W_C8, W_CNORMS8,
    W_SUBROWS, W_SUBID, W_SUBD, W_SUBOFF, W_MEMBERS2, W_SUBNN, W_SUBNND, W_SUBBASE, W_SUBCNT, W_CHAINPOS,
    W_LHIST, W_LOFFS, W_LSUMS, W_CAND, W_CANDCNT, W_HLIST, W_HCOUNT, W_STATS,
    W_OOC_A, W_OOC_B, W_OOC_C, W_OOC_D, W_OOC_E, W_OOC_F, W_OOC_G, W_CR, W_CRNORMS,
    W_KM_TRAIN, W_KM_MIND, W_KM_FLAG, W_KM_SEL, W_KM_POS, W_KM_SUMS, W_KM_NEW, W_KM_PSI, W_KM_P, W_KM_PN, W_KM_P8,
    W_KM_PN8, W_KM_OI, W_KM_OD, W_CH8, W_CHN, W_CHR, W_CHCNT, W_PAIRS, W_TOP2A, W_TOP2B, W_BUCKETD, W_KEY2,
    W_BYKEY, W_BKTD, W_BOFF, W_SUBPOS, W_TOP2H, W_RV1, W_RV1M, W_XH, W_UBASE, W_UROWS, W_UITEMS, W_TQ, W_SQ, W_PAIRS2, W_COUNT_
};
static_assert(W_COUNT_ <= 112, "workspace slots");

struct Ctx {
    gt_ctx* c;
    hipStream_t s;
    explicit Ctx(gt_ctx* cc) : c(cc), s(cc->stream) {}
    template <typename T> T* ws(int slot, size_t n) { return c->ws[slot].as<T>(n); }
    void sync() { GT_HIP(hipStreamSynchronize(s)); }
    void h2d(void* dst, const void* src, size_t bytes) {
        if (bytes) GT_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, s));
    }
    void d2h(void* dst, const void* src, size_t bytes) {
        if (bytes) GT_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, s));
    }
    void d2d(void* dst, const void* src, size_t bytes) {
        if (bytes && dst != src) GT_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, s));
    }
    // device view of a caller buffer: the pointer itself if it is device
    // memory, otherwise a workspace (uploaded when `upload`).
    template <typename T> T* in(int slot, const T* user, size_t n, bool upload = true) {
        if (is_device_ptr(user)) return const_cast<T*>(user);
        T* d = ws<T>(slot, n);
        if (upload) h2d(d, user, n * sizeof(T));
        return d;
    }
    template <typename T> void out(T* user, const T* dev, size_t n) {
        if (static_cast<const void*>(user) == static_cast<const void*>(dev)) return;
        if (is_device_ptr(user)) d2d(user, dev, n * sizeof(T));
        else d2h(user, dev, n * sizeof(T));
    }
    // device-event timing of the work enqueued by f
    template <typename F> double timed(F&& f) {
        GT_HIP(hipEventRecord(c->ev0, s));
        f();
        GT_HIP(hipEventRecord(c->ev1, s));
        GT_HIP(hipEventSynchronize(c->ev1));
        float ms = 0.f;
        GT_HIP(hipEventElapsedTime(&ms, c->ev0, c->ev1));
        return ms * 1e-3;
    }
};

static int pad_dim(int D) { return (D + 31) / 32 * 32; }

// longest list the fused kNN kernels keep per query
constexpr int kMaxListM = 128;

// Lays out work items XCD-major for knn_fused_kernel: groups of items (one
// group per bucket, sharing its pool) are dealt to the 8 XCDs longest-first
// onto the least-loaded XCD (cost = query rows x pool rows), each XCD runs
// its groups biggest-first, and every XCD list is padded with empty items to
// the same length.
static std::vector<WorkItem> layout_xcd(const std::vector<std::vector<WorkItem>>& groups)
{
    constexpr int kXcd = 8;
    std::vector<double> cost(groups.size(), 0.0);
    for (size_t g = 0; g < groups.size(); ++g)
        for (const WorkItem& it : groups[g]) cost[g] += static_cast<double>(it.q_count) * it.p_count;
    std::vector<size_t> order(groups.size());
    std::iota(order.begin(), order.end(), size_t(0));
    std::stable_sort(order.begin(), order.end(), [&](size_t x, size_t y) { return cost[x] > cost[y]; });
    std::vector<std::vector<WorkItem>> lists(kXcd);
    std::vector<double> load(kXcd, 0.0);
    for (size_t g : order) {
        const int x = static_cast<int>(std::min_element(load.begin(), load.end()) - load.begin());
        load[static_cast<size_t>(x)] += cost[g];
        lists[static_cast<size_t>(x)].insert(lists[static_cast<size_t>(x)].end(), groups[g].begin(), groups[g].end());
    }
    size_t per = 0;
    for (const auto& l : lists) per = std::max(per, l.size());
    WorkItem empty{};
    empty.q_count = 0;
    std::vector<WorkItem> out;
    out.reserve(per * kXcd);
    for (auto& l : lists) {
        l.resize(per, empty);
        out.insert(out.end(), l.begin(), l.end());
    }
    return out;
}

// layout_xcd for groups of one item each of (nearly) equal cost: dealt
// round-robin to the XCDs in order, lists padded to the same length.
static std::vector<WorkItem> layout_flat(const std::vector<WorkItem>& items)
{
    constexpr size_t kXcd = 8;
    const size_t per = (items.size() + kXcd - 1) / kXcd;
    WorkItem empty{};
    empty.q_count = 0;
    std::vector<WorkItem> out(per * kXcd, empty);
    for (size_t i = 0; i < items.size(); ++i) out[(i % kXcd) * per + i / kXcd] = items[i];
    return out;
}

static size_t dtype_size(int dtype)
{
    GT_REQUIRE(dtype == GT_DTYPE_F32 || dtype == GT_DTYPE_U8 || dtype == GT_DTYPE_I8, "unknown dtype");
    return dtype == GT_DTYPE_F32 ? 4 : 1;
}

struct DevMatrix {
    const float* data = nullptr;
    const float* norms = nullptr;
    int64_t N = 0;
    int D = 0;
    int Dp = 0;
    // int8 rows of integer-typed inputs (uint8 shifted by -shift), stride
    // Dp8 bytes, with their exact |x|^2; null for fp32 inputs unless every
    // value is an integer in [-128, 127] or [0, 255] (from_float)
    const int8_t* data8 = nullptr;
    const float* norms8 = nullptr;
    int Dp8 = 0;
    int shift = 0;
    bool from_float = false;
    // >= 0: every value is an integer in [-128, 127] + iv_shift (integer
    // inputs; float rows found integer-valued, with or without their int8 copy)
    int iv_shift = -1;
};

// The int8 kernel runs a (query, pool) pair when both sides have int8 rows
// with the same shift and the metric is unchanged by it (L2, or IP unshifted).
static bool use_i8(const DevMatrix& q, const DevMatrix& p, int metric)
{
    return q.data8 && p.data8 && q.shift == p.shift && q.Dp8 == p.Dp8 && (metric == GT_METRIC_L2 || q.shift == 0);
}

// padded fp32 device copy (or the caller's own device buffer when it already
// has that layout) plus row norms; with_i8: also int8 rows for integer inputs
// of at most 256 dimensions
// with_i8: also an int8 copy for the int8 matrix cores, for integer-typed
// inputs and (int_exact) for float inputs whose values are all integers in
// [-128, 127] or [0, 255] -- there every distance is an exact integer below
// 2^24 in both kernels, so the int8 kernel returns the fp32 kernel's keys.
static DevMatrix prepare(Ctx& c, int slot_x, int slot_raw, int slot_norms, const void* X, int64_t N, int D, int dtype,
                         bool with_i8 = false, bool int_exact = false)
{
    GT_REQUIRE(X != nullptr && N > 0 && D > 0, "empty dataset");
    GT_REQUIRE(N < (int64_t(1) << 31), "N must be < 2^31");
    if (slot_x == W_X) ++c.c->data_gen;   // the screen's fp16 copy of these rows is stale
    const int Dp = pad_dim(D);
    GT_REQUIRE(Dp <= 1024, "dimension > 1024 is not supported by this build");
    const size_t es = dtype_size(dtype);
    DevMatrix m;
    m.N = N;
    m.D = D;
    m.Dp = Dp;
    const bool dev = is_device_ptr(X);
    const void* src = X;   // device copy of the caller's rows
    if (with_i8 && (dtype == GT_DTYPE_U8 || dtype == GT_DTYPE_I8) && Dp <= 256) {
        // integer rows: float copy, int8 copy and both norms in one pass
        if (!dev) {
            void* raw = c.c->ws[slot_raw].ensure(static_cast<size_t>(N) * D * es);
            c.h2d(raw, X, static_cast<size_t>(N) * D * es);
            src = raw;
        }
        float* xp = c.ws<float>(slot_x, static_cast<size_t>(N) * Dp);
        float* nrm = c.ws<float>(slot_norms, static_cast<size_t>(N));
        int8_t* x8 = c.ws<int8_t>(W_X8, static_cast<size_t>(N) * Dp);
        float* n8 = c.ws<float>(W_NORMS8, static_cast<size_t>(N));
        launch_prepare_int(src, dtype, N, D, Dp, xp, nrm, x8, n8, c.s);
        m.data = xp;
        m.norms = nrm;
        m.Dp8 = Dp;
        m.shift = dtype == GT_DTYPE_U8 ? 128 : 0;
        m.iv_shift = m.shift;
        m.data8 = x8;
        m.norms8 = n8;
        return m;
    }
    if (dev && dtype == GT_DTYPE_F32 && D == Dp && (reinterpret_cast<uintptr_t>(X) & 15) == 0) {
        m.data = static_cast<const float*>(X);
    } else {
        if (!dev) {
            void* raw = c.c->ws[slot_raw].ensure(static_cast<size_t>(N) * D * es);
            c.h2d(raw, X, static_cast<size_t>(N) * D * es);
            src = raw;
        }
        float* xp = c.ws<float>(slot_x, static_cast<size_t>(N) * Dp);
        launch_pad_convert(src, dtype, xp, N, D, Dp, c.s);
        m.data = xp;
    }
    float* nrm = c.ws<float>(slot_norms, static_cast<size_t>(N));
    // float rows of a build: norms and the integer check in one pass (an
    // integer-valued dataset takes the exact int8 path with int_exact, and
    // its bucketing uses integer-rounded centroids either way)
    const bool check_int = with_i8 && dtype == GT_DTYPE_F32 && Dp <= 256;
    int* range = nullptr;
    if (check_int) {
        int* part = c.ws<int>(W_SUBD, static_cast<size_t>(3 * ((N + 3) / 4)));
        range = c.ws<int>(W_FLAG, 4);
        launch_row_norms_range(m.data, N, Dp, nrm, part, range, c.s);
    } else {
        launch_row_norms(m.data, N, Dp, nrm, c.s);
    }
    m.norms = nrm;
    if (with_i8 && (dtype == GT_DTYPE_U8 || dtype == GT_DTYPE_I8) && Dp <= 256) {
        m.Dp8 = Dp;
        m.shift = dtype == GT_DTYPE_U8 ? 128 : 0;
        m.iv_shift = m.shift;
        int8_t* x8 = c.ws<int8_t>(W_X8, static_cast<size_t>(N) * Dp);
        launch_pad_i8(src, dtype, x8, N, D, Dp, c.s);
        float* n8 = c.ws<float>(W_NORMS8, static_cast<size_t>(N));
        launch_row_norms_i8(x8, N, Dp, n8, c.s);
        m.data8 = x8;
        m.norms8 = n8;
    } else if (check_int) {
        int h[3];
        c.d2h(h, range, sizeof(h));   // padding columns are zeros: integers
        c.sync();
        const int shift = h[0] ? -1 : (h[1] >= -128 && h[2] <= 127) ? 0 : (h[1] >= 0 && h[2] <= 255) ? 128 : -1;
        m.iv_shift = shift;
        if (shift >= 0 && int_exact) {
            m.Dp8 = Dp;
            m.shift = shift;
            m.from_float = true;
            int8_t* x8 = c.ws<int8_t>(W_X8, static_cast<size_t>(N) * Dp);
            float* n8 = c.ws<float>(W_NORMS8, static_cast<size_t>(N));
            launch_quantize_norms_i8(m.data, N, D, Dp, shift, x8, n8, c.s);   // exact; padding 0
            m.data8 = x8;
            m.norms8 = n8;
        }
    }
    return m;
}

// Operands of one kNN launch: int8 rows where use_i8 allows, else fp32.
static void set_operands(KnnArgs& a, const DevMatrix& q, const DevMatrix& p, int metric)
{
    if (use_i8(q, p, metric)) {
        a.Xq8 = q.data8;
        a.Xp8 = p.data8;
        a.nq = q.norms8;
        a.np = p.norms8;
        a.Dp = q.Dp8;
    } else {
        a.Xq = q.data;
        a.Xp = p.data;
        a.nq = q.norms;
        a.np = p.norms;
        a.Dp = q.Dp;
    }
}

// Fused kNN of a query list against a pool list, optionally split over the
// pool for parallelism (partial lists merged afterwards).  Output rows:
// out_by_id ? query row id : query index.
struct KnnJob {
    const DevMatrix* Q;
    const DevMatrix* P;
    const int32_t* q_rows = nullptr;   // device, nullptr = identity
    int64_t nq = 0;
    const int32_t* p_rows = nullptr;   // device, nullptr = identity
    int64_t np = 0;
    int M = 0;
    int metric = 0;
    bool exclude_self = true;
    bool out_pos = false;
    int32_t* out_ids = nullptr;        // device (nq x M)
    float* out_d = nullptr;
};

static void run_knn_flat(Ctx& c, const KnnJob& j, int min_items = 2048)
{
    if (c.c->dbg.knn_resident) {
        // short lists of int8 rows against a small pool: the pool in LDS
        KnnArgs a{};
        set_operands(a, *j.Q, *j.P, j.metric);
        a.q_rows = j.q_rows;
        a.p_rows = j.p_rows;
        a.M = j.M;
        a.metric = j.metric;
        a.exclude_self = j.exclude_self ? 1 : 0;
        a.out_pos = j.out_pos ? 1 : 0;
        a.out_ids = j.out_ids;
        a.out_d = j.out_d;
        if (resident_supported(a, j.np)) {
            launch_knn_resident(a, j.nq, j.np, c.s);
            return;
        }
    }
    const int64_t qtiles = ceil_div(j.nq, kQueriesPerBlock);
    int splits = 1;
    if (qtiles < min_items && j.np > 4096) {
        const int64_t want = ceil_div(min_items, qtiles);
        const int64_t by_pool = j.np / 2048;
        splits = static_cast<int>(std::max<int64_t>(1, std::min<int64_t>({want, by_pool, 2048 / j.M, 64})));
    }
    const int64_t chunk = ceil_div(j.np, splits);
    std::vector<WorkItem> flat;
    flat.reserve(static_cast<size_t>(qtiles * splits));
    for (int s = 0; s < splits; ++s) {
        const int64_t p0 = s * chunk;
        const int64_t pc = std::min<int64_t>(chunk, j.np - p0);
        for (int64_t t = 0; t < qtiles; ++t) {
            WorkItem it;
            it.q_begin = t * kQueriesPerBlock;
            it.q_count = static_cast<int32_t>(std::min<int64_t>(kQueriesPerBlock, j.nq - it.q_begin));
            it.p_begin = p0;
            it.p_count = static_cast<int32_t>(std::max<int64_t>(pc, 0));
            it.out_base = static_cast<int64_t>(s) * j.nq + it.q_begin;
            flat.push_back(it);
        }
    }
    const std::vector<WorkItem> items = layout_flat(flat);
    WorkItem* d_items = c.ws<WorkItem>(W_ITEMS, items.size());
    c.h2d(d_items, items.data(), items.size() * sizeof(WorkItem));
    int32_t* oi = j.out_ids;
    float* od = j.out_d;
    if (splits > 1) {
        oi = c.ws<int32_t>(W_PART_I, static_cast<size_t>(splits) * j.nq * j.M);
        od = c.ws<float>(W_PART_D, static_cast<size_t>(splits) * j.nq * j.M);
    }
    KnnArgs a{};
    set_operands(a, *j.Q, *j.P, j.metric);
    a.q_rows = j.q_rows;
    a.p_rows = j.p_rows;
    a.items = d_items;
    a.n_items = static_cast<int32_t>(items.size());
    a.M = j.M;
    a.metric = j.metric;
    a.exclude_self = j.exclude_self ? 1 : 0;
    a.out_pos = j.out_pos ? 1 : 0;
    a.out_ids = oi;
    a.out_d = od;
    launch_knn_fused(a, c.s);
    if (splits > 1) launch_merge_partials(oi, od, j.nq, splits, j.M, j.out_ids, j.out_d, c.s);
}

// ---------------------------------------------------------------- bucketing

static uint64_t splitmix64(uint64_t& x)
{
    uint64_t z = (x += 0x9E3779B97F4A7C15ull);
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

// C distinct ids of [0, N), ascending (Floyd's sampling, seeded)
static std::vector<int32_t> sample_ids(int64_t N, int64_t C, uint64_t seed)
{
    // Floyd's sampling of C distinct ids of [0, N), membership in a bitmap
    std::vector<uint64_t> bits(static_cast<size_t>((N + 63) / 64), 0);
    auto test_set = [&](int64_t x) {
        uint64_t& w = bits[static_cast<size_t>(x >> 6)];
        const uint64_t m = 1ull << (x & 63);
        const bool had = (w & m) != 0;
        w |= m;
        return had;
    };
    uint64_t st = seed * 0x9E3779B97F4A7C15ull + 0x632BE59BD9B4E019ull;
    for (int64_t jj = N - C; jj < N; ++jj) {
        // uniform in [0, jj] by a 64 x 64 -> 128-bit multiply (Lemire's
        // reduction) instead of a 64-bit division
        const int64_t t = static_cast<int64_t>(
            (static_cast<unsigned __int128>(splitmix64(st)) * static_cast<uint64_t>(jj + 1)) >> 64);
        if (test_set(t)) test_set(jj);
    }
    std::vector<int32_t> ids;
    ids.reserve(static_cast<size_t>(C));
    for (size_t wi = 0; wi < bits.size(); ++wi)
        for (uint64_t w = bits[wi]; w; w &= w - 1)
            ids.push_back(static_cast<int32_t>(wi * 64 + static_cast<size_t>(__builtin_ctzll(w))));
    return ids;
}

// The random draws of one round's bucketing (host work that depends only on
// N, C and the seed, so a build draws every round's at its start, on a
// worker thread, while the dataset is prepared).
struct RoundSamples {
    std::vector<int32_t> cid;     // C centroid rows (uniform seeds; empty with KMeans||)
    std::vector<int32_t> srows;   // Lloyd training subset (empty without Lloyd)
    bool kmpar = false;           // seeds by KMeans|| on the device
    std::vector<int32_t> train;   // KMeans|| training rows, ascending
    int64_t first = 0;            // KMeans|| first candidate: index into train
    uint64_t seed = 0;            // KMeans|| device draws and final subsample
};

static int64_t lloyd_subset(int64_t N, int64_t C) { return std::min<int64_t>(N, std::max<int64_t>(65536, 256 * C)); }

// The KMeans|| training subset (src/bucket.cu:8857-8880): every row kept
// independently with probability frac (gaps between kept rows drawn from the
// geometric distribution, so the draw costs one step per kept row); all rows
// when frac >= 1 or when fewer than 4 C rows are kept.
static std::vector<int32_t> bernoulli_rows(int64_t N, int64_t C, double frac, uint64_t seed)
{
    std::vector<int32_t> rows;
    if (frac < 1.0) {
        uint64_t st = seed * 0x9E3779B97F4A7C15ull + 1;
        const double l1 = std::log1p(-frac);
        rows.reserve(static_cast<size_t>(static_cast<double>(N) * frac * 1.05) + 16);
        for (int64_t i = -1;;) {
            const double u = (static_cast<double>(splitmix64(st) >> 11) + 0.5) * (1.0 / 9007199254740992.0);
            const double gap = std::floor(std::log(u) / l1);
            if (!(gap < static_cast<double>(N))) break;
            i += 1 + static_cast<int64_t>(gap);
            if (i >= N) break;
            rows.push_back(static_cast<int32_t>(i));
        }
    }
    if (static_cast<int64_t>(rows.size()) < std::min<int64_t>(N, 4 * C) || frac >= 1.0) {
        rows.resize(static_cast<size_t>(N));
        std::iota(rows.begin(), rows.end(), 0);
    }
    return rows;
}

static bool seeds_by_kmpar(const gt_build_params& p)
{
    return p.seeding == GT_SEED_KMEANS_PAR || (p.seeding == GT_SEED_AUTO && p.kmeans_iters <= 0);
}

static RoundSamples draw_round(int64_t N, int64_t C, const gt_build_params& p, uint64_t seed)
{
    RoundSamples r;
    C = std::max<int64_t>(1, std::min<int64_t>(C, N));
    if (seeds_by_kmpar(p)) {
        // the reference pipeline trains on min(0.1, 1e7 / N) of the rows
        // (sk/scripts/dataset_env.py:57)
        const double frac = p.kmeans_train_fraction > 0.f ? static_cast<double>(p.kmeans_train_fraction)
                                                           : std::min(0.1, 1e7 / static_cast<double>(N));
        r.kmpar = true;
        r.seed = seed * 0xD1B54A32D192ED03ull + 0x5851F42D4C957F2Dull;
        r.train = bernoulli_rows(N, C, frac, seed);
        uint64_t st = r.seed;
        r.first = static_cast<int64_t>(splitmix64(st) % static_cast<uint64_t>(r.train.size()));
    } else {
        r.cid = sample_ids(N, C, seed);
    }
    if (p.kmeans_iters > 0) r.srows = sample_ids(N, lloyd_subset(N, C), seed * 0x2545F4914F6CDD1Dull + 7);
    return r;
}

struct Buckets {
    std::vector<int64_t> offsets;   // C+1
    PinnedI32 members;              // N
    std::vector<int32_t> probe;     // C x P (bucket indices, -1 = none)
    int P = 0;
    uint64_t gen = 0;               // which bucketing (0: none recorded)
    hipEvent_t uploaded = nullptr;  // recorded after each upload of members, if set
};

// generation of a host bucketing, never 0
static uint64_t next_bucket_gen()
{
    static std::atomic<uint64_t> g{0};
    return ++g;
}

// Two-choice assignment (src/bucket.cu:2276-2302): point i goes to its 2nd
// nearest centroid if that bucket is smaller than balance x the nearest
// one's, sizes counted in point order.  Centroids that are data points sit
// in their own bucket from the start.
template <typename T>
static void assign_two_choice(const T* top2, int64_t N, int64_t C, float balance,
                              const std::vector<int32_t>* centroid_ids, int32_t* bucket_of)
{
    std::fill(bucket_of, bucket_of + N, -1);
    std::vector<int64_t> size(static_cast<size_t>(C), 0);
    if (centroid_ids) {
        for (int64_t c = 0; c < C; ++c) {
            bucket_of[static_cast<size_t>((*centroid_ids)[static_cast<size_t>(c)])] = static_cast<int32_t>(c);
            size[static_cast<size_t>(c)] = 1;
        }
    }
    // every nearest centroid valid (checked before the sequential loop)
    bool bad = false;
    for (int64_t i = 0; i < N; ++i) bad |= top2[static_cast<size_t>(2 * i)] >= static_cast<uint64_t>(C);
    GT_REQUIRE(!bad, "top-2 assignment returned an invalid centroid");
    const double bal = balance > 0.f ? static_cast<double>(balance) : -1.0;   // -1: never the second
    int64_t* sz = size.data();
    for (int64_t i = 0; i < N; ++i) {
        if (bucket_of[i] >= 0) continue;
        const uint32_t c1 = top2[static_cast<size_t>(2 * i)];
        const uint32_t c2 = top2[static_cast<size_t>(2 * i + 1)];
        // branch-free: the second centroid's size read at c1 when it is missing
        const bool ok2 = c2 < static_cast<uint64_t>(C);
        const uint32_t c2s = ok2 ? c2 : c1;
        const bool take = ok2 && static_cast<double>(sz[c2s]) < bal * static_cast<double>(sz[c1]);
        const uint32_t chosen = take ? c2 : c1;
        bucket_of[i] = static_cast<int32_t>(chosen);
        sz[chosen]++;
    }
}

// Process-wide pool of host worker threads (created once, never torn down:
// the threads only ever run host code).  run(T, f) calls f(t) for t in
// [0, T), t = 0 on the caller, and returns when all have finished; parallel
// regions of different callers are serialised.
class HostPool {
public:
    static HostPool& get()
    {
        static HostPool* p = new HostPool();
        return *p;
    }
    int size() const { return T_; }
    template <typename F>
    void run(int T, F&& f)
    {
        if (T <= 1) {
            f(0);
            return;
        }
        std::lock_guard<std::mutex> one(run_m_);
        std::function<void(int)> job = [&](int t) { f(t); };
        {
            std::lock_guard<std::mutex> lk(m_);
            job_ = &job;
            ntask_ = T;
            next_ = 1;
            pending_ = T - 1;
        }
        cv_.notify_all();
        f(0);
        std::unique_lock<std::mutex> lk(m_);
        done_.wait(lk, [&] { return pending_ == 0; });
        job_ = nullptr;
    }

private:
    HostPool() : T_(static_cast<int>(std::max(1u, std::min(16u, std::thread::hardware_concurrency()))))
    {
        for (int i = 1; i < T_; ++i) std::thread([this] { loop(); }).detach();
    }
    void loop()
    {
        std::unique_lock<std::mutex> lk(m_);
        for (;;) {
            cv_.wait(lk, [&] { return job_ != nullptr && next_ < ntask_; });
            const int t = next_++;
            std::function<void(int)>* job = job_;
            lk.unlock();
            (*job)(t);
            lk.lock();
            if (--pending_ == 0) done_.notify_all();
        }
    }
    int T_;
    std::mutex run_m_, m_;
    std::condition_variable cv_, done_;
    std::function<void(int)>* job_ = nullptr;
    int ntask_ = 0, next_ = 0, pending_ = 0;
};

// Runs f(t, lo, hi) over T contiguous slices of [0, n).
template <typename F>
static void parallel_slices(int64_t n, int T, F&& f)
{
    if (T <= 1 || n < 65536) {
        f(0, int64_t(0), n);
        return;
    }
    HostPool::get().run(T, [&](int t) { f(t, n * t / T, n * (t + 1) / T); });
}

static int host_threads() { return HostPool::get().size(); }

// Stable counting sort: out = in ordered by key[in[e]] (keys in [0, K)),
// equal keys keep their order; off (K+1) receives the key offsets.  Each
// thread counts and scatters its own slice, so the order is the serial one.
static void counting_sort(const int32_t* in, int64_t n, const int32_t* key, int64_t K, int32_t* out,
                          std::vector<int64_t>& off)
{
    const int T = n < 65536 ? 1 : host_threads();
    std::vector<int64_t> cnt(static_cast<size_t>(T) * static_cast<size_t>(K), 0);
    parallel_slices(n, T, [&](int t, int64_t lo, int64_t hi) {
        int64_t* c = cnt.data() + static_cast<size_t>(t) * K;
        for (int64_t e = lo; e < hi; ++e) c[key[in ? in[e] : e]]++;
    });
    off.assign(static_cast<size_t>(K + 1), 0);
    int64_t run = 0;
    for (int64_t k = 0; k < K; ++k) {
        off[static_cast<size_t>(k)] = run;
        for (int t = 0; t < T; ++t) {
            int64_t& c = cnt[static_cast<size_t>(t) * K + k];
            const int64_t v = c;
            c = run;
            run += v;
        }
    }
    off[static_cast<size_t>(K)] = run;
    parallel_slices(n, T, [&](int t, int64_t lo, int64_t hi) {
        int64_t* c = cnt.data() + static_cast<size_t>(t) * K;
        for (int64_t e = lo; e < hi; ++e) {
            const int32_t v = in ? in[e] : static_cast<int32_t>(e);
            out[c[key[v]]++] = v;
        }
    });
}

// Stable counting sort of positions e in [0, n) by key[e] (keys in [0, K)):
// out[pos] = val ? val[e] : e, and out_carry[pos] = carry[e] when carry is
// given; off (K+1) receives the key offsets.  Each thread counts and
// scatters its own slice, so the order is the serial one.
static void counting_sort_kv(const int32_t* key, const int32_t* val, int64_t n, int64_t K, int32_t* out,
                             const int32_t* carry, int32_t* out_carry, std::vector<int64_t>& off)
{
    const int T = n < 65536 ? 1 : host_threads();
    std::vector<int64_t> cnt(static_cast<size_t>(T) * static_cast<size_t>(K), 0);
    parallel_slices(n, T, [&](int t, int64_t lo, int64_t hi) {
        int64_t* c = cnt.data() + static_cast<size_t>(t) * K;
        for (int64_t e = lo; e < hi; ++e) c[key[e]]++;
    });
    off.assign(static_cast<size_t>(K + 1), 0);
    int64_t run = 0;
    for (int64_t k = 0; k < K; ++k) {
        off[static_cast<size_t>(k)] = run;
        for (int t = 0; t < T; ++t) {
            int64_t& c = cnt[static_cast<size_t>(t) * K + k];
            const int64_t v = c;
            c = run;
            run += v;
        }
    }
    off[static_cast<size_t>(K)] = run;
    parallel_slices(n, T, [&](int t, int64_t lo, int64_t hi) {
        int64_t* c = cnt.data() + static_cast<size_t>(t) * K;
        for (int64_t e = lo; e < hi; ++e) {
            const int64_t pos = c[key[e]]++;
            out[pos] = val ? val[e] : static_cast<int32_t>(e);
            if (carry) out_carry[pos] = carry[e];
        }
    });
}

// CSR of an assignment with members ordered by (bucket, key2, id): two stable
// counting sorts.  key2 = each point's other top-2 centroid, so that points
// of one bucket near the same neighbouring bucket sit next to each other.
static void csr_from_assignment_keyed(const int32_t* bucket_of, int64_t N, const std::vector<int32_t>& key2,
                                      int64_t C, Buckets& b, std::vector<int32_t>& by_key, std::vector<int32_t>& bkt)
{
    by_key.resize(static_cast<size_t>(N));
    bkt.resize(static_cast<size_t>(N));
    std::vector<int64_t> off;
    // the ids by key2, each carrying its bucket, then by bucket: both passes
    // read their keys in order
    counting_sort_kv(key2.data(), nullptr, N, C, by_key.data(), bucket_of, bkt.data(), off);
    b.members.resize(static_cast<size_t>(N));
    counting_sort_kv(bkt.data(), by_key.data(), N, C, b.members.data(), nullptr, nullptr, b.offsets);
}

// Orders each bucket's members by their nearest sub-centroid (every
// kSubSize-th member of the bucket, by the fused kernel with lists of one),
// the sub-centroids themselves along a greedy nearest-neighbour chain: an
// unseeded pass that starts one sub-centroid's worth of rows before a
// query's own tile then meets the query's nearest rows first (its own
// sub-cluster and the two beside it on the chain), so its threshold tightens
// within a few tiles and few candidates reach the list merges.  The kNN
// result does not depend on the order of the pool.
constexpr int kSubSize = 128;     // members per sub-centroid
constexpr int kSubMax = 1024;     // sub-centroids per bucket (LDS counters of the sort)
static void sub_order_members(Ctx& c, const DevMatrix& X, const Buckets& b, int metric, int32_t* d_members)
{
    const int64_t C = static_cast<int64_t>(b.offsets.size()) - 1;
    const int64_t N = X.N;
    std::vector<int32_t> subrows;
    std::vector<std::vector<WorkItem>> groups(static_cast<size_t>(C)), sgroups(static_cast<size_t>(C));
    std::vector<int64_t> sbase(static_cast<size_t>(C), 0);
    std::vector<int32_t> scount(static_cast<size_t>(C), 0);
    bool any = false;
    for (int64_t bb = 0; bb < C; ++bb) {
        const int64_t lo = b.offsets[static_cast<size_t>(bb)], n = b.offsets[static_cast<size_t>(bb + 1)] - lo;
        if (n < 2 * kSubSize) continue;   // left as it is (the sort copies it)
        const int64_t s = std::min<int64_t>(kSubMax, ceil_div(n, kSubSize));
        const int64_t p0 = static_cast<int64_t>(subrows.size());
        sbase[static_cast<size_t>(bb)] = p0;
        scount[static_cast<size_t>(bb)] = static_cast<int32_t>(s);
        for (int64_t i = 0; i < s; ++i) subrows.push_back(static_cast<int32_t>(lo + i * n / s));   // positions
        for (int64_t t = 0; t < s; t += kQueriesPerBlock) {   // sub-centroids among themselves
            WorkItem it;
            it.q_begin = p0 + t;
            it.q_count = static_cast<int32_t>(std::min<int64_t>(kQueriesPerBlock, s - t));
            it.p_begin = p0;
            it.p_count = static_cast<int32_t>(s);
            it.p_rot = 0;
            it.out_base = p0 + t;
            sgroups[static_cast<size_t>(bb)].push_back(it);
        }
        for (int64_t t = 0; t < n; t += kQueriesPerBlock) {
            WorkItem it;
            it.q_begin = lo + t;
            it.q_count = static_cast<int32_t>(std::min<int64_t>(kQueriesPerBlock, n - t));
            it.p_begin = p0;
            it.p_count = static_cast<int32_t>(s);
            it.p_rot = 0;
            it.out_base = lo + t;   // one key per member position
            groups[static_cast<size_t>(bb)].push_back(it);
        }
        any = true;
    }
    if (!any) return;
    // the sub-centroid rows: the members at those positions (d_members holds
    // this bucketing's members in its own order)
    int32_t* d_subpos = c.ws<int32_t>(W_SUBPOS, subrows.size());
    c.h2d(d_subpos, subrows.data(), subrows.size() * sizeof(int32_t));
    int32_t* d_sub = c.ws<int32_t>(W_SUBROWS, subrows.size());
    launch_gather_i32(d_members, d_subpos, static_cast<int64_t>(subrows.size()), d_sub, c.s);
    const std::vector<WorkItem> items = layout_xcd(groups);
    WorkItem* d_items = c.ws<WorkItem>(W_ITEMS, items.size());
    c.h2d(d_items, items.data(), items.size() * sizeof(WorkItem));
    int32_t* d_key = c.ws<int32_t>(W_SUBID, static_cast<size_t>(N));
    float* d_kd = c.ws<float>(W_SUBD, static_cast<size_t>(N));
    KnnArgs a{};
    set_operands(a, X, X, metric);
    a.q_rows = d_members;
    a.p_rows = d_sub;
    a.items = d_items;
    a.n_items = static_cast<int32_t>(items.size());
    a.M = 1;
    a.metric = metric;
    a.exclude_self = 0;
    a.out_pos = 1;   // sub-centroid index within the bucket
    a.out_ids = d_key;
    a.out_d = d_kd;
    launch_knn_fused(a, c.s);

    // each sub-centroid's nearest sub-centroids of its bucket (itself among
    // them), then the chain
    constexpr int kChainK = 9;
    const int64_t ns = static_cast<int64_t>(subrows.size());
    const std::vector<WorkItem> sitems = layout_xcd(sgroups);
    WorkItem* d_sitems = c.ws<WorkItem>(W_TASKS, sitems.size());
    c.h2d(d_sitems, sitems.data(), sitems.size() * sizeof(WorkItem));
    int32_t* d_nn = c.ws<int32_t>(W_SUBNN, static_cast<size_t>(ns) * kChainK);
    float* d_nnd = c.ws<float>(W_SUBNND, static_cast<size_t>(ns) * kChainK);
    KnnArgs sa = a;
    sa.q_rows = d_sub;
    sa.items = d_sitems;
    sa.n_items = static_cast<int32_t>(sitems.size());
    sa.M = kChainK;
    sa.out_ids = d_nn;
    sa.out_d = d_nnd;
    launch_knn_fused(sa, c.s);
    int64_t* d_sbase = c.ws<int64_t>(W_SUBBASE, static_cast<size_t>(C));
    c.h2d(d_sbase, sbase.data(), static_cast<size_t>(C) * sizeof(int64_t));
    int32_t* d_scount = c.ws<int32_t>(W_SUBCNT, static_cast<size_t>(C));
    c.h2d(d_scount, scount.data(), static_cast<size_t>(C) * sizeof(int32_t));
    int32_t* d_chain = c.ws<int32_t>(W_CHAINPOS, static_cast<size_t>(ns));
    launch_sub_chain(d_nn, kChainK, d_sbase, d_scount, C, d_chain, c.s);

    int64_t* d_off = c.ws<int64_t>(W_SUBOFF, static_cast<size_t>(C + 1));
    c.h2d(d_off, b.offsets.data(), static_cast<size_t>(C + 1) * sizeof(int64_t));
    int32_t* d_m2 = c.ws<int32_t>(W_MEMBERS2, static_cast<size_t>(N));
    launch_segment_sort(d_members, d_key, d_off, C, 2 * kSubSize, d_chain, d_sbase, d_m2, c.s);
    c.d2d(d_members, d_m2, static_cast<size_t>(N) * sizeof(int32_t));
}

// One round of pooled kNN into (out_ids, out_d) rows by global id.
// seed_d (device, optional) caps kept keys at the running M-th distance.
// own / probes select the pool segments: the bucket's own members and the
// members of its probe buckets (both by default).
// With b1 >= 0 only buckets [b0, b1) run and their members' lists go to
// compact rows (member position - offsets[b0]), seeded from the same rows
// (the out-of-core build's chunks).
static double bucketed_round(Ctx& c, const DevMatrix& X, const Buckets& b, int M, int metric, const float* seed_d,
                             int32_t* out_ids, float* out_d, int64_t* max_pool, int64_t* max_bucket,
                             double* pairs, bool own = true, bool probes = true, int64_t b0 = 0, int64_t b1 = -1,
                             int32_t* run_ids = nullptr, bool* merged = nullptr)
{
    const int64_t C = static_cast<int64_t>(b.offsets.size()) - 1;
    const int64_t N = X.N;
    const bool compact = b1 >= 0;
    if (!compact) b1 = C;
    GT_REQUIRE(b0 >= 0 && b0 <= b1 && b1 <= C, "bucket range out of bounds");
    const int64_t qbase = b.offsets[static_cast<size_t>(b0)];
    const int64_t rows = compact ? b.offsets[static_cast<size_t>(b1)] - qbase : N;
    Trace tr;
    std::vector<CopyTaskH> tasks;
    // every pool starts at a multiple of kChunkRows in the pool list (the
    // collect kernel's pruning chunks); pool_cnt: its rows
    std::vector<int64_t> pool_off(static_cast<size_t>(C + 1), 0), pool_cnt(static_cast<size_t>(C), 0);
    int64_t total = 0;
    std::vector<int64_t> segs;
    for (int64_t bb = b0; bb < b1; ++bb) {
        total = ceil_div(total, int64_t(kChunkRows)) * kChunkRows;
        pool_off[static_cast<size_t>(bb)] = total;
        segs.clear();
        if (own) segs.push_back(bb);
        for (int p = 0; probes && p < b.P; ++p) {
            const int64_t pb = b.probe[static_cast<size_t>(bb * b.P + p)];
            if (pb < 0 || pb >= C || pb == bb) continue;
            if (std::find(segs.begin(), segs.end(), pb) != segs.end()) continue;
            segs.push_back(pb);
        }
        for (int64_t sb : segs) {
            const int64_t lo = b.offsets[static_cast<size_t>(sb)], n = b.offsets[static_cast<size_t>(sb + 1)] - lo;
            if (n == 0) continue;
            tasks.push_back({lo, total, n});
            total += n;
        }
        pool_cnt[static_cast<size_t>(bb)] = total - pool_off[static_cast<size_t>(bb)];
    }
    pool_off[static_cast<size_t>(b1)] = total;

    // the members go up once per bucketing: a later pass over the same
    // buckets finds them in place (perhaps reordered within each bucket by
    // the sub-centroid order, which changes no result)
    int32_t* d_members = c.ws<int32_t>(W_MEMBERS, static_cast<size_t>(N));
    if (b.gen == 0 || c.c->members_gen != b.gen) {
        GT_REQUIRE(static_cast<int64_t>(b.members.size()) == N, "bucket members are on the device only");
        c.h2d(d_members, b.members.data(), static_cast<size_t>(N) * sizeof(int32_t));
        if (b.uploaded) GT_HIP(hipEventRecord(b.uploaded, c.s));
        c.c->members_gen = b.gen;
    }
    // members by nearest sub-centroid: for the unseeded pass (its threshold
    // tightens within a few tiles), and for seeded passes that prune chunks
    // (a chunk of 64 consecutive members then lies within one sub-cluster,
    // and so do a block's 128 queries: small spheres, few chunks needed)
    const bool want_prune = metric == GT_METRIC_L2 && X.data8 && c.c->dbg.knn_prune != 0 && c.c->dbg.knn_collect != 0 &&
                            (X.Dp8 == 32 || X.Dp8 == 64 || X.Dp8 == 128 || X.Dp8 == 256);
    // and for seeded passes the fp16 screen cuts (each work item's union of
    // candidate rows is then a few sub-clusters, not the whole pool; the
    // unseeded pass is sub-ordered either way)
    // (knn_screen 1: passes of at least 2^27 pairs, below which its launches
    // cost more than it saves -- C1's 10^7-pair passes measured 0.1 ms slower
    // each; 2: every pass it can take)
    double pairs_all = 0.0;
    for (int64_t bb = b0; bb < b1; ++bb)
        pairs_all += static_cast<double>(b.offsets[static_cast<size_t>(bb + 1)] - b.offsets[static_cast<size_t>(bb)]) *
                     static_cast<double>(pool_cnt[static_cast<size_t>(bb)]);
    const int scr = c.c->dbg.knn_screen;
    const bool want_screen = c.c->dbg.knn_collect != 0 && !use_i8(X, X, metric) &&
                             (scr == 2 || (scr == 1 && pairs_all >= static_cast<double>(int64_t(1) << 27)));
    const bool sub_ordered = own && !compact && c.c->dbg.sub_order != 0 && (!seed_d || want_prune || want_screen);
    if (sub_ordered) sub_order_members(c, X, b, metric, d_members);
    CopyTaskH* d_tasks = c.ws<CopyTaskH>(W_TASKS, tasks.size());
    c.h2d(d_tasks, tasks.data(), tasks.size() * sizeof(CopyTaskH));
    int32_t* d_pool = c.ws<int32_t>(W_POOL, static_cast<size_t>(std::max<int64_t>(total, 1)));
    launch_copy_ranges(d_tasks, static_cast<int64_t>(tasks.size()), d_members, d_pool, c.s);

    std::vector<std::vector<WorkItem>> groups(static_cast<size_t>(C));
    int64_t mp = 0, mb = 0;
    double pr = 0.0;
    for (int64_t bb = b0; bb < b1; ++bb) {
        const int64_t q0 = b.offsets[static_cast<size_t>(bb)], nqb = b.offsets[static_cast<size_t>(bb + 1)] - q0;
        const int64_t p0 = pool_off[static_cast<size_t>(bb)], npb = pool_cnt[static_cast<size_t>(bb)];
        mp = std::max(mp, npb);
        mb = std::max(mb, nqb);
        pr += static_cast<double>(nqb) * static_cast<double>(npb);
        for (int64_t t = 0; t < nqb; t += kQueriesPerBlock) {
            WorkItem it;
            it.q_begin = q0 + t;
            it.q_count = static_cast<int32_t>(std::min<int64_t>(kQueriesPerBlock, nqb - t));
            it.p_begin = p0;
            it.p_count = static_cast<int32_t>(npb);
            // own bucket = first pool segment: start the scan at these queries'
            // own rows (members are ordered so that neighbours sit close by),
            // for the sub-ordered unseeded pass one sub-cluster earlier (the
            // chain's previous sub-cluster lies there)
            int64_t rot = own && npb > 0 ? t : 0;
            if (sub_ordered && !seed_d && nqb >= 2 * kSubSize && npb >= kSubSize) rot = (t - kSubSize + npb) % npb;   // >= 0
            GT_REQUIRE(rot >= 0 && (npb == 0 || rot < npb), "pool rotation out of range");
            it.p_rot = static_cast<int32_t>(rot);
            it.out_base = compact ? q0 - qbase + t : -1;
            groups[static_cast<size_t>(bb)].push_back(it);
        }
    }
    GT_REQUIRE(mp < (int64_t(1) << 31), "pool too large");
    const std::vector<WorkItem> items = layout_xcd(groups);
    WorkItem* d_items = c.ws<WorkItem>(W_ITEMS, items.size());
    c.h2d(d_items, items.data(), items.size() * sizeof(WorkItem));

    tr.mark(c.s, "round: pools + work items");
    KnnArgs a{};
    set_operands(a, X, X, metric);
    a.q_rows = d_members;
    a.p_rows = d_pool;
    a.items = d_items;
    a.n_items = static_cast<int32_t>(items.size());
    a.M = M;
    a.metric = metric;
    a.exclude_self = 1;
    a.out_pos = 0;
    a.seed_d = seed_d;
    a.seed_ld = M;
    a.out_ids = out_ids;
    a.out_d = out_d;
    // lists of at most 64 keys on int8 rows: collect + select (every point
    // is the query of exactly one work item, so rows = N)
    const bool collect = c.c->dbg.knn_collect != 0 && knn_collect_supported(a);
    if (collect) {
        // (+ one wave's rows of slack: the selection reads whole groups of
        // 32 rows and masks the rows past the last)
        a.cand = c.ws<uint64_t>(W_CAND, static_cast<size_t>(rows + kQueriesPerWave) * kCollectCap);
        a.cand_cnt = c.ws<int32_t>(W_CANDCNT, static_cast<size_t>(rows));
        if (tr.on && c.c->dbg.knn_stats) {   // counters of the collect launch (slow), printed below
            a.stats = c.ws<unsigned long long>(W_STATS, 8);
            GT_HIP(hipMemsetAsync(a.stats, 0, 8 * sizeof(unsigned long long), c.s));
        }
        a.pairs_done = c.ws<unsigned long long>(W_PAIRS, 1);
        GT_HIP(hipMemsetAsync(a.pairs_done, 0, sizeof(unsigned long long), c.s));
        // a seeded pass given its running table's ids: the new lists merge
        // into (run_ids, seed_d) in place
        if (run_ids && seed_d) {
            a.run_ids = run_ids;
            a.run_d = const_cast<float*>(seed_d);
            a.hl_rows = c.ws<int32_t>(W_HLIST, static_cast<size_t>(rows));
            a.hl_count = c.ws<uint32_t>(W_HCOUNT, 1);
        }
    }
    if (merged) *merged = a.run_ids != nullptr;
    // the unseeded pass's threshold window: 32 tiles on large builds (C5:
    // 423 -> about 200 keys per query, kNN 97 -> 80 ms), 16 below (C2: 32
    // tiles take 0.14 ms more than the 23 % fewer keys save)
    a.window_tiles = c.c->dbg.knn_window > 0 ? c.c->dbg.knn_window : X.N >= (int64_t(1) << 22) ? 32 : 16;
    // fp16 screen on fp32 rows: each work item's pool cut to the rows whose
    // fp16 key, less a bound on its gap to the fp32 key, is at or below some
    // query's threshold -- the running M-th distance of a seeded pass, else
    // a bound on the pool's M-th smallest key from the screen's own window
    // -- a superset of the rows the fp32 pass keeps, so its lists are
    // unchanged; the fp32 pass then scans each item's union (items and pool
    // list replaced)
    bool screen = want_screen && collect && a.Xq && !a.Xq8 && screen_supported(a.Dp, mp);
    // the screen's own window: 16 tiles (C3: 32, 64 and 128 tiles shrink
    // the union by 1.7, 3.5 and 6.5 % and cost more than that saves); the
    // fp32 pass over the unions takes 32 (C3 kNN 22.9 -> 21.9 ms)
    const int screen_window = a.window_tiles;
    if (screen && c.c->dbg.knn_window <= 0) a.window_tiles = 32;
    int64_t* d_ubase = nullptr;
    int32_t* d_urows = nullptr;
    WorkItem* d_uitems = nullptr;
    uint16_t* d_xh = nullptr;
    float* d_tq = nullptr;
    int32_t* d_pairs = nullptr;
    int n_pairs = 0;
    if (screen) {
        std::vector<int64_t> ub(items.size(), 0);
        int64_t u = 0;
        for (size_t i = 0; i < items.size(); ++i) {
            ub[i] = u;
            if (items[i].q_count > 0) u += items[i].p_count;
        }
        screen = u < (int64_t(1) << 30);   // the union list's room: every item's whole pool
        if (screen) {
            d_ubase = c.ws<int64_t>(W_UBASE, ub.size());
            c.h2d(d_ubase, ub.data(), ub.size() * sizeof(int64_t));
            d_urows = c.ws<int32_t>(W_UROWS, static_cast<size_t>(std::max<int64_t>(u, 1)));
            d_uitems = c.ws<WorkItem>(W_UITEMS, items.size());
            d_xh = c.ws<uint16_t>(W_XH, static_cast<size_t>(N) * X.Dp);
            a.items = d_uitems;
            a.p_rows = d_urows;
            // the screen's pairs: consecutive items with queries and the same
            // pool (a bucket's items sit together), padded to a multiple of 8
            std::vector<int32_t> pr;
            int32_t held = -1;
            for (size_t i = 0; i < items.size(); ++i) {
                if (items[i].q_count <= 0) continue;
                if (held >= 0 && items[static_cast<size_t>(held)].p_begin == items[i].p_begin &&
                    items[static_cast<size_t>(held)].p_count == items[i].p_count) {
                    pr.push_back(held);
                    pr.push_back(static_cast<int32_t>(i));
                    held = -1;
                } else {
                    if (held >= 0) { pr.push_back(held); pr.push_back(-1); }
                    held = static_cast<int32_t>(i);
                }
            }
            if (held >= 0) { pr.push_back(held); pr.push_back(-1); }
            while ((pr.size() / 2) % 8 != 0) { pr.push_back(-1); pr.push_back(-1); }
            n_pairs = static_cast<int>(pr.size() / 2);
            d_pairs = c.ws<int32_t>(W_PAIRS2, std::max<size_t>(pr.size(), 2));
            c.h2d(d_pairs, pr.data(), pr.size() * sizeof(int32_t));
            // an unseeded pass's bounds serve the screen only: the fp32 pass
            // takes its own (exact, tighter) window from each union,
            // rotated to the queries' own rows
            if (!seed_d) d_tq = c.ws<float>(W_TQ, static_cast<size_t>(std::max<int64_t>(rows, 1)));
        }
    }
    // exact chunk pruning (int8 rows, L2): the centre and radius of every
    // kChunkRows rows of the pool list
    const bool prune = collect && a.Xq8 && a.Xp8 && metric == GT_METRIC_L2 && c.c->dbg.knn_prune != 0 &&
                       (X.Dp8 == 32 || X.Dp8 == 64 || X.Dp8 == 128 || X.Dp8 == 256);
    int64_t nchunk = 0;
    int32_t* d_chcnt = nullptr;
    if (prune) {
        nchunk = ceil_div(total, int64_t(kChunkRows));
        std::vector<int32_t> cnt(static_cast<size_t>(std::max<int64_t>(nchunk, 1)), 0);
        for (int64_t bb = b0; bb < b1; ++bb) {
            const int64_t g0 = pool_off[static_cast<size_t>(bb)] / kChunkRows, n = pool_cnt[static_cast<size_t>(bb)];
            for (int64_t k = 0; k * kChunkRows < n; ++k)
                cnt[static_cast<size_t>(g0 + k)] = static_cast<int32_t>(std::min<int64_t>(kChunkRows, n - k * kChunkRows));
        }
        d_chcnt = c.ws<int32_t>(W_CHCNT, cnt.size());
        c.h2d(d_chcnt, cnt.data(), cnt.size() * sizeof(int32_t));
        a.ch8 = c.ws<int8_t>(W_CH8, static_cast<size_t>(std::max<int64_t>(nchunk, 1)) * X.Dp8);
        a.chn = c.ws<float>(W_CHN, static_cast<size_t>(std::max<int64_t>(nchunk, 1)));
        a.chr = c.ws<float>(W_CHR, static_cast<size_t>(std::max<int64_t>(nchunk, 1)));
    }
    const double done_before = c.c->knn_pairs_done;
    const double t = c.timed([&] {
        if (prune)
            launch_chunk_bounds(X.data8, X.Dp8, d_pool, d_chcnt, nchunk, const_cast<int8_t*>(a.ch8),
                                const_cast<float*>(a.chn), const_cast<float*>(a.chr), c.s);
        if (screen) {
            // the fp16 copy once per prepared dataset (every pass of a build
            // screens the same rows)
            unsigned int* d_sq = c.ws<unsigned int>(W_SQ, 1);
            if (c.c->screen_gen != c.c->data_gen || c.c->screen_src != X.data) {
                launch_screen_prepare(X.data, X.norms, N, X.Dp, d_sq, d_xh, c.s);
                c.c->screen_gen = c.c->data_gen;
                c.c->screen_src = X.data;
            }
            launch_screen(d_items, a.n_items, d_pairs, n_pairs, d_ubase, d_members, d_pool, d_xh, X.norms, d_sq, X.Dp,
                          metric, seed_d, M, M,
                          screen_window, d_tq, d_urows, d_uitems, a.pairs_done, c.s);
        }
        if (collect) launch_knn_collect_select(a, rows, c.s);
        else launch_knn_fused(a, c.s);
    });
    if (tr.on && screen) {
        std::vector<WorkItem> ui(items.size());
        c.d2h(ui.data(), d_uitems, ui.size() * sizeof(WorkItem));
        c.sync();
        double up = 0.0, pp = 0.0;
        for (size_t i = 0; i < ui.size(); ++i) {
            if (ui[i].q_count <= 0) continue;
            up += ui[i].p_count;
            pp += items[i].p_count;
        }
        std::fprintf(stderr, "[gtann]   screen: %.4g of %.4g item pool rows kept (%.2f %%)\n", up, pp,
                     100.0 * up / std::max(pp, 1.0));
    }
    // the collect kernels on int8 rows and the screen count the pairs their
    // MFMAs computed; the fp32 collect kernel computes every pair
    if (a.pairs_done && (a.Xq8 || screen)) {
        unsigned long long done = 0;
        c.d2h(&done, a.pairs_done, sizeof(done));
        c.sync();
        c.c->knn_pairs_done += static_cast<double>(done);
    } else {
        c.c->knn_pairs_done += pr;
    }
    ++c.c->knn_launches;
    tr.mark(c.s, "round: fused kNN");
    if (tr.on)
        std::fprintf(stderr, "[gtann]   pairs %.4g, computed %.4g (own %d, probes %d, seeded %d), %.3f ms device\n", pr,
                     a.pairs_done ? c.c->knn_pairs_done - done_before : pr, own ? 1 : 0, probes ? 1 : 0,
                     seed_d ? 1 : 0, t * 1e3);
    if (tr.on && a.stats) {
        unsigned long long h[8];
        c.d2h(h, a.stats, sizeof(h));
        c.sync();
        std::fprintf(stderr, "[gtann]   collect: %.3g keys (%.1f per query), %llu compactions, %.3g of %.3g wave tiles past the pre-filter\n",
                     static_cast<double>(h[0]), static_cast<double>(h[0]) / static_cast<double>(N), h[1],
                     static_cast<double>(h[2]), static_cast<double>(h[3]));
        if (a.run_ids)
            std::fprintf(stderr, "[gtann]   merge: %llu rows with keys, %.3g fresh keys, %llu rows with fresh keys, %llu with more than M\n",
                         h[4], static_cast<double>(h[5]), h[6], h[7]);
    }
    if (max_pool) *max_pool = std::max(*max_pool, mp);
    if (max_bucket) *max_bucket = std::max(*max_bucket, mb);
    if (pairs) *pairs += pr;
    return t;
}

// The device half of one round's bucketing: centroids (sampled rows, moved by
// the Lloyd iterations), every point's exact top-2 centroids downloaded into
// pinned host memory, the probe table and the optional centroid self-kNN.
// The host half (bucket_host) only reads this plan, so it can run on another
// thread while the device works on the next round.
struct BucketPlan {
    int64_t N = 0, C = 0;
    std::vector<int32_t> cid;       // sampled centroid row ids, ascending
    bool data_points = true;        // centroids are data points (no Lloyd)
    const uint32_t* top2 = nullptr; // pinned, 2N: nearest and 2nd nearest centroid (C >= 65535)
    const uint16_t* top2h = nullptr;    // the same as 16-bit ids (C < 65535; a missing one is 0xFFFF)
    const uint32_t* d_top2 = nullptr;   // the same on the device (the round's own buffer), or null
    std::vector<int32_t> probe;     // C x P
    int P = 0;
};

// KMeans|| seeds (src/bucket.cu:2833-3168): C distinct data points.  The
// first candidate is a uniform training row; in each of 3 rounds every
// training row that is not yet a candidate is taken with probability
// l * C * d^2 / psi (l = 0.5, so about 1.5 C candidates over the rounds;
// d = L2 distance to the nearest candidate, psi estimated from every
// (S / 16384)-th row, src/bucket.cu:2933-2935, 3003-3016), and the new
// candidates lower the distances (fused kNN, lists of one).  Then C of the
// candidates are chosen uniformly (src/bucket.cu:3134-3168).  Where the
// rounds leave C or fewer candidates the reference keeps them all and
// builds fewer buckets; here uniform training rows that are not candidates
// fill the C (the bucket count is a build parameter).  Returns the rows
// ascending.
static std::vector<int32_t> kmeans_par_seeds(Ctx& c, const DevMatrix& X, int64_t C, const RoundSamples& d)
{
    constexpr int kRounds = 3;
    constexpr double kOversample = 1.5 / kRounds;
    constexpr int64_t kPsiRows = 16384;
    const int64_t S = static_cast<int64_t>(d.train.size());
    GT_REQUIRE(S >= C && d.first >= 0 && d.first < S, "KMeans||: training subset smaller than the bucket count");
    int32_t* d_train = c.ws<int32_t>(W_KM_TRAIN, static_cast<size_t>(S));
    c.h2d(d_train, d.train.data(), static_cast<size_t>(S) * sizeof(int32_t));
    float* mind = c.ws<float>(W_KM_MIND, static_cast<size_t>(S));
    uint8_t* flag = c.ws<uint8_t>(W_KM_FLAG, static_cast<size_t>(S));
    uint32_t* sel = c.ws<uint32_t>(W_KM_SEL, static_cast<size_t>(S));
    uint32_t* pos = c.ws<uint32_t>(W_KM_POS, static_cast<size_t>(S) + 1);
    uint32_t* sums = c.ws<uint32_t>(W_KM_SUMS, static_cast<size_t>(ceil_div(S, int64_t(1024)) + 2));
    int32_t* d_new = c.ws<int32_t>(W_KM_NEW, static_cast<size_t>(S));
    float* psi = c.ws<float>(W_KM_PSI, 1);
    float* dnew = c.ws<float>(W_KM_OD, static_cast<size_t>(S));
    int32_t* oi = c.ws<int32_t>(W_KM_OI, static_cast<size_t>(S));
    launch_kmpar_init(flag, mind, S, d.first, c.s);
    // the distances of every training row to the candidates of d_new[0..n)
    auto lower = [&](int64_t n) {
        DevMatrix P;
        P.N = n;
        P.D = X.D;
        P.Dp = X.Dp;
        float* rows = c.ws<float>(W_KM_P, static_cast<size_t>(n) * X.Dp);
        float* norms = c.ws<float>(W_KM_PN, static_cast<size_t>(n));
        launch_gather_rows_f32(X.data, X.Dp, d_new, n, rows, c.s);
        launch_row_norms(rows, n, X.Dp, norms, c.s);
        P.data = rows;
        P.norms = norms;
        if (X.data8) {
            int8_t* r8 = c.ws<int8_t>(W_KM_P8, static_cast<size_t>(n) * X.Dp8);
            float* n8 = c.ws<float>(W_KM_PN8, static_cast<size_t>(n));
            launch_quantize_i8(rows, n, X.D, X.Dp8, X.shift, r8, c.s);   // exact: the rows are data points
            launch_row_norms_i8(r8, n, X.Dp8, n8, c.s);
            P.data8 = r8;
            P.norms8 = n8;
            P.Dp8 = X.Dp8;
            P.shift = X.shift;
            P.from_float = X.from_float;
        }
        P.iv_shift = X.iv_shift;
        KnnJob j;
        j.Q = &X;
        j.P = &P;
        j.q_rows = d_train;
        j.nq = S;
        j.np = n;
        j.M = 1;
        j.metric = GT_METRIC_L2;
        j.exclude_self = false;
        j.out_pos = true;
        j.out_ids = oi;
        j.out_d = dnew;
        run_knn_flat(c, j, 1);
        launch_kmpar_min(mind, dnew, S, c.s);
    };
    std::vector<int32_t> cand{d.train[static_cast<size_t>(d.first)]};
    c.h2d(d_new, cand.data(), sizeof(int32_t));
    lower(1);
    const float lk = static_cast<float>(kOversample * static_cast<double>(C));
    for (int it = 0; it < kRounds; ++it) {
        launch_kmpar_psi(mind, S, kPsiRows, psi, c.s);
        launch_kmpar_sample(mind, flag, sel, S, psi, lk, d.seed + static_cast<uint64_t>(it + 1) * 0xA0761D6478BD642Full,
                            c.s);
        launch_exclusive_scan(sel, S, pos, sums, c.s);
        launch_kmpar_compact(sel, pos, d_train, S, d_new, c.s);
        uint32_t n_new = 0;
        c.d2h(&n_new, pos + S, sizeof(n_new));
        c.sync();
        if (n_new == 0) break;
        const size_t old = cand.size();
        cand.resize(old + n_new);
        c.d2h(cand.data() + old, d_new, static_cast<size_t>(n_new) * sizeof(int32_t));
        if (it + 1 < kRounds) lower(n_new);
        c.sync();
    }
    uint64_t st = d.seed ^ 0x6A09E667F3BCC909ull;
    std::vector<int32_t> cid;
    if (static_cast<int64_t>(cand.size()) > C) {
        // C of the candidates, uniformly (a partial Fisher-Yates shuffle)
        for (int64_t i = 0; i < C; ++i) {
            const int64_t j = i + static_cast<int64_t>(splitmix64(st) % static_cast<uint64_t>(cand.size() - i));
            std::swap(cand[static_cast<size_t>(i)], cand[static_cast<size_t>(j)]);
        }
        cid.assign(cand.begin(), cand.begin() + C);
    } else {
        // every candidate, then uniform training rows that are not candidates
        cid = cand;
        std::vector<uint8_t> taken(static_cast<size_t>(S), 0);
        for (int32_t r : cand)
            taken[static_cast<size_t>(std::lower_bound(d.train.begin(), d.train.end(), r) - d.train.begin())] = 1;
        std::vector<int32_t> rest;
        rest.reserve(static_cast<size_t>(S) - cand.size());
        for (int64_t i = 0; i < S; ++i)
            if (!taken[static_cast<size_t>(i)]) rest.push_back(d.train[static_cast<size_t>(i)]);
        for (int64_t i = 0; static_cast<int64_t>(cid.size()) < C; ++i) {
            const int64_t j = i + static_cast<int64_t>(splitmix64(st) % static_cast<uint64_t>(rest.size() - i));
            std::swap(rest[static_cast<size_t>(i)], rest[static_cast<size_t>(j)]);
            cid.push_back(rest[static_cast<size_t>(i)]);
        }
    }
    std::sort(cid.begin(), cid.end());
    return cid;
}

static void bucket_device(Ctx& c, const DevMatrix& X, int64_t C, int nprobe, int metric, int kmeans_iters,
                          RoundSamples&& draws, HostBuf& pin, BucketPlan& bp, int parity,
                          std::vector<int32_t>* cknn = nullptr, int cknn_k = 0)
{
    const int64_t N = X.N;
    Trace tr;
    C = std::max<int64_t>(1, std::min<int64_t>(C, N));
    bp.N = N;
    bp.C = C;
    bp.cid = draws.kmpar ? kmeans_par_seeds(c, X, C, draws) : std::move(draws.cid);
    std::vector<int32_t>& cid = bp.cid;
    GT_REQUIRE(static_cast<int64_t>(cid.size()) == C, "centroid draw");
    int32_t* d_cid = c.ws<int32_t>(W_PROWS, static_cast<size_t>(C));
    c.h2d(d_cid, cid.data(), static_cast<size_t>(C) * sizeof(int32_t));

    // centroid matrix: the sampled rows themselves, optionally moved to the
    // means of their members by Lloyd iterations
    DevMatrix Cm;
    Cm.N = C;
    Cm.Dp = X.Dp;
    float* d_cm = c.ws<float>(W_C, static_cast<size_t>(C) * X.Dp);
    float* d_cn = c.ws<float>(W_CNORMS, static_cast<size_t>(C));
    // gather centroid rows via the pool-copy kernel on a float view: row r of
    // X is Dp floats; copy as int32 words (bit-exact)
    {
        std::vector<CopyTaskH> tasks(static_cast<size_t>(C));
        for (int64_t k = 0; k < C; ++k)
            tasks[static_cast<size_t>(k)] = {static_cast<int64_t>(cid[static_cast<size_t>(k)]) * X.Dp, k * X.Dp, X.Dp};
        CopyTaskH* d_tasks = c.ws<CopyTaskH>(W_TASKS, tasks.size());
        c.h2d(d_tasks, tasks.data(), tasks.size() * sizeof(CopyTaskH));
        launch_copy_ranges(d_tasks, C, reinterpret_cast<const int32_t*>(X.data), reinterpret_cast<int32_t*>(d_cm),
                           c.s);
    }
    launch_row_norms(d_cm, C, X.Dp, d_cn, c.s);
    Cm.N = C;
    Cm.D = X.D;
    Cm.data = d_cm;
    Cm.norms = d_cn;
    // an integer-valued dataset's assignment runs against the centroids
    // rounded to the dataset's values (the buckets only need near
    // centroids; every distance is then an exact integer): on the int8
    // kernel when the rows have their int8 copy, else on the fp32 kernel
    // with the same rounded centroids, so that the buckets do not depend on
    // which kernel runs
    float* d_cr = X.iv_shift >= 0 && !X.data8 ? c.ws<float>(W_CR, static_cast<size_t>(C) * X.Dp) : nullptr;
    float* d_crn = d_cr ? c.ws<float>(W_CRNORMS, static_cast<size_t>(C)) : nullptr;
    auto refresh_c8 = [&]() {
        if (X.iv_shift < 0) return;   // float data: fp32 centroids
        if (!X.data8) {
            launch_round_to_int(d_cm, C, X.D, X.Dp, X.iv_shift, d_cr, c.s);
            launch_row_norms(d_cr, C, X.Dp, d_crn, c.s);
            Cm.data = d_cr;
            Cm.norms = d_crn;
            return;
        }
        int8_t* c8 = c.ws<int8_t>(W_C8, static_cast<size_t>(C) * X.Dp8);
        float* cn8 = c.ws<float>(W_CNORMS8, static_cast<size_t>(C));
        launch_quantize_i8(d_cm, C, X.D, X.Dp8, X.shift, c8, c.s);
        launch_row_norms_i8(c8, C, X.Dp8, cn8, c.s);
        Cm.data8 = c8;
        Cm.norms8 = cn8;
        Cm.Dp8 = X.Dp8;
        Cm.shift = X.shift;
    };
    refresh_c8();
    tr.mark(c.s, "bucketing: sample centroids");

    // Lloyd iterations on a training subset (the reference's KMeans|| also
    // trains on a subset, src/bucket.cu:8857-8880): nearest centroid of every
    // sampled row, then each centroid moves to the mean of its sampled members.
    const bool data_points = kmeans_iters <= 0;
    if (!data_points) {
        const int64_t S = lloyd_subset(N, C);
        const std::vector<int32_t> srows = std::move(draws.srows);
        GT_REQUIRE(static_cast<int64_t>(srows.size()) == S, "Lloyd subset draw");
        int32_t* d_srows = c.ws<int32_t>(W_QROWS, static_cast<size_t>(S));
        c.h2d(d_srows, srows.data(), static_cast<size_t>(S) * sizeof(int32_t));
        int32_t* d_n1 = c.ws<int32_t>(W_IDS3, static_cast<size_t>(S));
        float* d_n1d = c.ws<float>(W_D3, static_cast<size_t>(S));
        // pinned staging: nearest (S) | members (S) | offsets (C + 1, int64)
        const size_t s4 = (static_cast<size_t>(S) * 4 + 7) / 8 * 8;
        char* pin = c.c->pin_lloyd.as<char>(2 * s4 + static_cast<size_t>(C + 1) * 8);
        int32_t* nearest = reinterpret_cast<int32_t*>(pin);
        int32_t* hmem = reinterpret_cast<int32_t*>(pin + s4);
        int64_t* hoff = reinterpret_cast<int64_t*>(pin + 2 * s4);
        int32_t* d_mem = c.ws<int32_t>(W_MEMBERS, static_cast<size_t>(S));
        c.c->members_gen = 0;   // W_MEMBERS no longer holds a bucketing's members
        int64_t* d_off = c.ws<int64_t>(W_OFF, static_cast<size_t>(C + 1));
        std::vector<int64_t> off;
        // the CSR on the device: no host round trip per iteration
        const bool host_csr = c.c->dbg.lloyd_host_csr != 0 || C > 16384;
        const int64_t nh = C * csr_blocks(S);
        uint32_t* d_lhist = host_csr ? nullptr : c.ws<uint32_t>(W_LHIST, static_cast<size_t>(nh));
        uint32_t* d_loffs = host_csr ? nullptr : c.ws<uint32_t>(W_LOFFS, static_cast<size_t>(nh + 1));
        uint32_t* d_lsums = host_csr ? nullptr : c.ws<uint32_t>(W_LSUMS, static_cast<size_t>(nh / 1024 + 2));
        for (int it = 0; it < kmeans_iters; ++it) {
            KnnJob j;
            j.Q = &X;
            j.P = &Cm;
            j.q_rows = d_srows;
            j.nq = S;
            j.np = C;
            j.M = 1;
            j.metric = metric;
            j.exclude_self = false;
            j.out_pos = true;
            j.out_ids = d_n1;
            j.out_d = d_n1d;
            run_knn_flat(c, j, 1);
            if (!host_csr) {
                // CSR in sample order (stable counting sort), members as row ids
                launch_sample_csr(d_n1, d_srows, S, static_cast<int>(C), d_lhist, d_loffs, d_lsums, d_mem, d_off, c.s);
            } else {
                c.d2h(nearest, d_n1, static_cast<size_t>(S) * sizeof(int32_t));
                c.sync();
                counting_sort(nullptr, S, nearest, C, hmem, off);
                parallel_slices(S, host_threads(), [&](int, int64_t lo, int64_t hi) {
                    for (int64_t e = lo; e < hi; ++e) hmem[e] = srows[static_cast<size_t>(hmem[e])];
                });
                std::copy(off.begin(), off.end(), hoff);
                c.h2d(d_mem, hmem, static_cast<size_t>(S) * sizeof(int32_t));
                c.h2d(d_off, hoff, static_cast<size_t>(C + 1) * sizeof(int64_t));
            }
            launch_centroid_sums(X.data, X.Dp, d_mem, d_off, C, d_cm, c.s);
            launch_row_norms(d_cm, C, X.Dp, d_cn, c.s);
            refresh_c8();
            tr.mark(c.s, "bucketing: Lloyd iteration");
        }
    }

    bp.data_points = data_points;

    // probe table: nprobe nearest other centroids
    bp.P = static_cast<int>(std::min<int64_t>(nprobe, C - 1));
    bp.probe.assign(static_cast<size_t>(C) * std::max(bp.P, 0), -1);
    if (bp.P > kMaxListM) {
        // wider than a kernel list (the reference allows nprobe up to 256):
        // exact top-P of the centroid distances on the host, (distance, id) order
        std::vector<float> hc(static_cast<size_t>(C) * X.Dp);
        c.d2h(hc.data(), d_cm, hc.size() * sizeof(float));
        c.sync();
        parallel_slices(C, std::min<int64_t>(host_threads(), C), [&](int, int64_t lo, int64_t hi) {
            std::vector<std::pair<double, int32_t>> row(static_cast<size_t>(C - 1));
            for (int64_t q = lo; q < hi; ++q) {
                const float* xq = hc.data() + q * X.Dp;
                size_t n = 0;
                for (int64_t o = 0; o < C; ++o) {
                    if (o == q) continue;
                    const float* xo = hc.data() + o * X.Dp;
                    double d = 0.0;
                    for (int k = 0; k < X.Dp; ++k) {
                        if (metric == GT_METRIC_IP) d -= static_cast<double>(xq[k]) * xo[k];
                        else d += (static_cast<double>(xq[k]) - xo[k]) * (static_cast<double>(xq[k]) - xo[k]);
                    }
                    row[n++] = {d, static_cast<int32_t>(o)};
                }
                std::partial_sort(row.begin(), row.begin() + bp.P, row.begin() + static_cast<std::ptrdiff_t>(n));
                for (int p = 0; p < bp.P; ++p)
                    bp.probe[static_cast<size_t>(q * bp.P + p)] = row[static_cast<size_t>(p)].second;
            }
        });
    } else if (bp.P > 0) {
        int32_t* d_pi = c.ws<int32_t>(W_PROBE_I, static_cast<size_t>(C) * bp.P);
        float* d_pd = c.ws<float>(W_PROBE_D, static_cast<size_t>(C) * bp.P);
        KnnJob j;
        j.Q = &Cm;
        j.P = &Cm;
        j.nq = C;
        j.np = C;
        j.M = bp.P;
        j.metric = metric;
        j.exclude_self = true;
        j.out_pos = true;
        j.out_ids = d_pi;
        j.out_d = d_pd;
        run_knn_flat(c, j, 1);
        c.d2h(bp.probe.data(), d_pi, bp.probe.size() * sizeof(int32_t));
        c.sync();
    }
    tr.mark(c.s, "bucketing: probe table");
    if (cknn && cknn_k > 0) {
        // exact self-kNN of the centroids (self excluded), centroid indices
        GT_REQUIRE(cknn_k <= C - 1 && cknn_k <= 128, "centroid_knn_k must be <= min(buckets - 1, 128)");
        int32_t* d_ki = c.ws<int32_t>(W_PROBE_I, static_cast<size_t>(C) * cknn_k);
        float* d_kd = c.ws<float>(W_PROBE_D, static_cast<size_t>(C) * cknn_k);
        KnnJob j;
        j.Q = &Cm;
        j.P = &Cm;
        j.nq = C;
        j.np = C;
        j.M = cknn_k;
        j.metric = metric;
        j.exclude_self = true;
        j.out_pos = true;
        j.out_ids = d_ki;
        j.out_d = d_kd;
        run_knn_flat(c, j, 1);
        cknn->resize(static_cast<size_t>(C) * cknn_k);
        c.d2h(cknn->data(), d_ki, cknn->size() * sizeof(int32_t));
        c.sync();
    }
    // exact top-2 centroids of every point, last: the host half starts as
    // soon as they are down (16-bit ids when the centroids allow)
    uint32_t* top2 = nullptr;
    bp.top2 = nullptr;
    bp.top2h = nullptr;
    bp.d_top2 = nullptr;
    const bool h16 = C < 65535;
    if (h16) bp.top2h = pin.as<uint16_t>(static_cast<size_t>(2 * N));
    else bp.top2 = top2 = pin.as<uint32_t>(static_cast<size_t>(2 * N));
    if (C >= 2) {
        // (each round parity its own buffer: the device CSR of a round reads
        // it after the next round's centroids are computed)
        int32_t* d_t2 = c.ws<int32_t>(parity ? W_TOP2B : W_TOP2A, static_cast<size_t>(2 * N));
        bp.d_top2 = reinterpret_cast<const uint32_t*>(d_t2);
        float* d_t2d = c.ws<float>(W_D3, static_cast<size_t>(2 * N));
        KnnJob j;
        j.Q = &X;
        j.P = &Cm;
        j.nq = N;
        j.np = C;
        j.M = 2;
        j.metric = metric;
        j.exclude_self = false;
        j.out_pos = true;
        j.out_ids = d_t2;
        j.out_d = d_t2d;
        run_knn_flat(c, j, 1);
        tr.mark(c.s, "bucketing: top-2 kNN");
        if (h16) {
            uint16_t* d_h = c.ws<uint16_t>(W_TOP2H, static_cast<size_t>(2 * N));
            launch_pack_u16(reinterpret_cast<const uint32_t*>(d_t2), 2 * N, d_h, c.s);
            c.d2h(const_cast<uint16_t*>(bp.top2h), d_h, static_cast<size_t>(2 * N) * sizeof(uint16_t));
        } else {
            c.d2h(top2, d_t2, static_cast<size_t>(2 * N) * sizeof(uint32_t));
        }
        c.sync();
        tr.mark(c.s, "bucketing: top-2 download");
    } else {
        uint16_t* th = const_cast<uint16_t*>(bp.top2h);
        for (int64_t i = 0; i < N; ++i) {
            if (h16) {
                th[2 * i] = 0;
                th[2 * i + 1] = 0xFFFF;
            } else {
                top2[2 * i] = 0u;
                top2[2 * i + 1] = 0xffffffffu;
            }
        }
    }
}

// The host half: two-choice rule over the downloaded top-2 lists into
// bucket_of (N), then, with csr, the members ordered by (bucket, other top-2
// centroid, id) (without it the device orders them: launch_bucket_csr).
// Host code only (no HIP calls), so the build runs it on a worker thread.
static void bucket_host(const BucketPlan& bp, float balance, Buckets& b, int32_t* bucket_of, bool csr,
                        std::vector<int32_t>& key2, std::vector<int32_t>& by_key, std::vector<int32_t>& bkt)
{
    const int64_t N = bp.N, C = bp.C;
    Trace tr;
    if (bp.top2h) assign_two_choice(bp.top2h, N, C, balance, bp.data_points ? &bp.cid : nullptr, bucket_of);
    else assign_two_choice(bp.top2, N, C, balance, bp.data_points ? &bp.cid : nullptr, bucket_of);
    const double t_tc = tr.t.sec();
    b.P = bp.P;
    b.probe = bp.probe;
    b.gen = next_bucket_gen();
    if (!csr) {
        b.members.clear();   // the members live on the device only
        if (tr.on) std::fprintf(stderr, "[gtann] bucketing (host thread): two-choice %.3f ms\n", t_tc * 1e3);
        return;
    }
    key2.resize(static_cast<size_t>(N));
    parallel_slices(N, host_threads(), [&](int, int64_t lo, int64_t hi) {
        for (int64_t i = lo; i < hi; ++i) {
            const size_t e = static_cast<size_t>(2 * i);
            const uint32_t c1 = bp.top2h ? bp.top2h[e] : bp.top2[e], c2 = bp.top2h ? bp.top2h[e + 1] : bp.top2[e + 1];
            const uint32_t other = static_cast<int64_t>(c1) == bucket_of[static_cast<size_t>(i)] ? c2 : c1;
            key2[static_cast<size_t>(i)] = other < static_cast<uint64_t>(C) ? static_cast<int32_t>(other)
                                                                              : bucket_of[static_cast<size_t>(i)];
        }
    });
    csr_from_assignment_keyed(bucket_of, N, key2, C, b, by_key, bkt);
    if (tr.on)
        std::fprintf(stderr, "[gtann] bucketing (host thread): two-choice %.3f ms, CSR %.3f ms\n", t_tc * 1e3,
                     (tr.t.sec() - t_tc) * 1e3);
}

// ---------------------------------------------------------------- graph stages

// Each graph stage is enqueued (kernels only, no host round trip, so that a
// caller's events around it time the device work) and its flag is checked
// after.  The flags are cleared by a kernel.
struct StageFlags {
    unsigned long long* bad = nullptr;   // prune: lowest row with too few candidates, ~0 if none
    int* err = nullptr;                  // reverse merge: an id >= N
};

static StageFlags stage_flags(Ctx& c)
{
    StageFlags f;
    f.bad = c.ws<unsigned long long>(W_FLAG, 1);
    f.err = c.ws<int>(W_TMP, 1);
    return f;
}

// order: a permutation of the rows to process them in (rows that share
// neighbours close together keep those rows in L2), or null
static void prune_enqueue(Ctx& c, const StageFlags& f, const int32_t* G, int64_t N, int M, int K, uint32_t* out,
                          const int32_t* order = nullptr)
{
    GT_REQUIRE(K >= 1 && K <= M, "output degree must be in [1, M]");
    launch_init_flags(f.bad, f.err, c.s);
    launch_cagra_prune(G, N, M, K, out, f.bad, c.s, order, c.c->dbg.prune_flat_rows != 0);
}

static void prune_check(Ctx& c, const StageFlags& f)
{
    unsigned long long h = 0;
    c.d2h(&h, f.bad, sizeof(h));
    c.sync();
    if (h != ~0ull)
        throw Error(GT_EFEWCAND, "prune: row " + std::to_string(h) +
                                     " has fewer than output_degree valid candidates");
}

static void prune_device(Ctx& c, const int32_t* G, int64_t N, int M, int K, uint32_t* out)
{
    const StageFlags f = stage_flags(c);
    prune_enqueue(c, f, G, N, M, K, out);
    prune_check(c, f);
}

static void reverse_merge_enqueue(Ctx& c, const StageFlags& f, const uint32_t* fwd, int64_t N, int K, uint32_t* out,
                                  int forced = -1)
{
    GT_REQUIRE(K >= 1 && K <= 64, "output degree must be in [1, 64]");
    GT_REQUIRE(N * K < (int64_t(1) << 32), "too many edges for 32-bit offsets");
    int* err = f.err;
    launch_init_flags(f.bad, f.err, c.s);
    // Four paths give the same rows: the two-kernel merge over block-local
    // key regions (2^8-row bins, output degree <= 48: graphs up to 2^21
    // rows), the same merge behind a level of superbins (larger graphs), the
    // binned merge through global grouping (up to 2^26 rows; degrees above
    // 48), the global-atomic CSR merge beyond.  The context's revmerge_path
    // forces one (tests).
    if (forced < 0) forced = c.c->dbg.revmerge_path;
    RvPlan rp{};
    const int shift = forced == 3 ? -1 : rev_bin_shift(N);
    bool use_rv = false;
    if (forced == 1) {
        use_rv = rv_plan(N, K, rp);
    } else if (forced == 4) {
        use_rv = rv_plan2(N, K, rp);
    } else if (forced == 0 && K <= 48) {
        use_rv = rv_plan(N, K, rp) && rp.cshift == 8;
        if (!use_rv) use_rv = rv_plan2(N, K, rp);
    }
    if (use_rv) {
        const RvSizes z = rv_sizes(N, K, rp);
        RvBufs bf;
        bf.part = c.ws<uint32_t>(W_KEYS, z.part);
        bf.meta_blk = reinterpret_cast<uint16_t*>(c.ws<uint32_t>(W_DEG, (z.meta + 1) / 2));
        bf.meta = reinterpret_cast<uint16_t*>(c.ws<uint32_t>(W_OFF, (z.meta + 1) / 2));
        if (rp.two) {
            bf.part1 = c.ws<uint32_t>(W_RV1, z.part1);
            bf.meta1 = reinterpret_cast<uint16_t*>(c.ws<uint32_t>(W_RV1M, (z.meta1 + 1) / 2));
        }
        uint32_t* slow = c.ws<uint32_t>(W_CUR, static_cast<size_t>(N) + 1);   // [0]: count, then rows
        uint32_t* big = c.ws<uint32_t>(W_SUMS, static_cast<size_t>(rp.nbins) + 1);   // [0]: count, then bins
        launch_rv(fwd, N, K, rp, bf, out, err, slow + 1, slow, big, c.s);
    } else if (shift >= 0) {
        // binned path: LDS histograms and cursors, no global atomics
        const int64_t nh = ceil_div(N, int64_t(1) << shift) * rev_bin_blocks(N * K);
        uint32_t* hist = c.ws<uint32_t>(W_DEG, static_cast<size_t>(nh));
        uint32_t* offs = c.ws<uint32_t>(W_OFF, static_cast<size_t>(nh + 1));
        uint32_t* sums = c.ws<uint32_t>(W_SUMS, static_cast<size_t>(ceil_div(nh, 1024) + 1));
        unsigned long long* part = c.ws<unsigned long long>(W_KEYS, static_cast<size_t>(N * K));
        unsigned long long* grouped = c.ws<unsigned long long>(W_CUR, static_cast<size_t>(N * K));
        launch_rev_binned(fwd, N, K, hist, offs, sums, part, grouped, out, err, c.s);
    } else {
        uint32_t* deg = c.ws<uint32_t>(W_DEG, static_cast<size_t>(N));
        uint32_t* off = c.ws<uint32_t>(W_OFF, static_cast<size_t>(N + 1));
        uint32_t* slot = c.ws<uint32_t>(W_CUR, static_cast<size_t>(N * K));
        uint32_t* sums = c.ws<uint32_t>(W_SUMS, static_cast<size_t>(ceil_div(N, 1024) + 1));
        unsigned long long* keys = c.ws<unsigned long long>(W_KEYS, static_cast<size_t>(N * K));
        GT_HIP(hipMemsetAsync(deg, 0, static_cast<size_t>(N) * sizeof(uint32_t), c.s));
        launch_rev_count(fwd, N, K, deg, slot, err, c.s);
        launch_exclusive_scan(deg, N, off, sums, c.s);
        launch_rev_scatter(fwd, N, K, off, slot, keys, c.s);
        launch_rev_merge(fwd, N, K, off, keys, out, c.s);
    }
}

// Reads the merge's error word after reverse_merge_enqueue: 1 = an id >= N;
// 2 = a level-two block of the two-level merge held more keys than it takes
// (destinations concentrated in one superbin), whose rows are then redone by
// the binned merge.  Returns the seconds of that redo.
static double reverse_merge_check(Ctx& c, const StageFlags& f, const uint32_t* fwd, int64_t N, int K, uint32_t* out)
{
    int h = 0;
    c.d2h(&h, f.err, sizeof(int));
    c.sync();
    double t = 0.0;
    if (h == 2) {
        t = c.timed([&] { reverse_merge_enqueue(c, f, fwd, N, K, out, 2); });
        c.d2h(&h, f.err, sizeof(int));
        c.sync();
    }
    if (h) throw Error(GT_EINVAL, "reverse merge: forward graph holds an id >= N");
    return t;
}

static void reverse_merge_device(Ctx& c, const uint32_t* fwd, int64_t N, int K, uint32_t* out)
{
    const StageFlags f = stage_flags(c);
    reverse_merge_enqueue(c, f, fwd, N, K, out);
    reverse_merge_check(c, f, fwd, N, K, out);
}

// bd/build_bucket.py:473-543 on a device table (N x M, ascending rows), in place
static void reverse_insert_device(Ctx& c, int32_t* ids, float* d, int64_t N, int M)
{
    GT_REQUIRE(M >= 1 && M <= 128, "list length must be in [1, 128]");
    GT_REQUIRE(N * M < (int64_t(1) << 32), "too many edges for 32-bit offsets");
    const int64_t E = N * M;
    float* worst = c.ws<float>(W_WORST, static_cast<size_t>(N));
    uint32_t* cnt = c.ws<uint32_t>(W_DEG, static_cast<size_t>(N));
    uint32_t* off = c.ws<uint32_t>(W_OFF, static_cast<size_t>(N + 1));
    uint32_t* slot = c.ws<uint32_t>(W_CUR, static_cast<size_t>(E));
    uint32_t* sums = c.ws<uint32_t>(W_SUMS, static_cast<size_t>(ceil_div(N, 1024) + 1));
    unsigned long long* keys = c.ws<unsigned long long>(W_KEYS, static_cast<size_t>(E));
    int* err = c.ws<int>(W_TMP, 1);
    GT_HIP(hipMemsetAsync(cnt, 0, static_cast<size_t>(N) * sizeof(uint32_t), c.s));
    GT_HIP(hipMemsetAsync(err, 0, sizeof(int), c.s));
    launch_rin_worst(d, N, M, worst, c.s);
    launch_rin_count(ids, d, N, M, worst, cnt, slot, err, c.s);
    launch_exclusive_scan(cnt, N, off, sums, c.s);
    launch_rin_scatter(ids, d, N, M, off, slot, keys, c.s);
    launch_rin_merge(ids, d, N, M, off, keys, c.s);
    int h = 0;
    c.d2h(&h, err, sizeof(int));
    c.sync();
    if (h) throw Error(GT_EINVAL, "reverse-edge insertion: table holds an id >= N");
}

// ---------------------------------------------------------------- out-of-core stages
// The N x M table and the N x K graphs stay in host memory; one chunk at a
// time goes through a device budget (bytes of device memory for the chunk's
// buffers; the dataset, when a stage needs it, is not counted).  Every stage
// gives the same rows as its resident counterpart.

// src/optimize.cu:89-134 on a host table (the rule of sanitize_kernel), rows
// in parallel.
static void sanitize_host(const int32_t* in, int64_t N, int M, uint32_t* out)
{
    parallel_slices(N, host_threads(), [&](int, int64_t lo, int64_t hi) {
        for (int64_t i = lo; i < hi; ++i) {
            const int32_t* r = in + i * M;
            uint32_t* o = out + i * M;
            int first = -1;
            for (int k = 0; k < M && first < 0; ++k)
                if (r[k] >= 0 && r[k] < N && r[k] != i) first = k;
            const uint32_t fb = first < 0 ? static_cast<uint32_t>((i + 1) % N) : static_cast<uint32_t>(r[first]);
            for (int k = 0; k < M; ++k)
                o[k] = (r[k] < 0 || r[k] >= N || r[k] == i) ? fb : static_cast<uint32_t>(r[k]);
        }
    });
}

struct OocReport {
    int64_t chunks = 0;         // device chunks of the stage
    double rows_moved = 0.0;    // table rows sent to the device
};

// Exact CAGRA prune (cagra_prune_kernel) of a sanitized host table san
// (N x M) into host rows out (N x K).  Rows go in chunks; a chunk's device
// table holds its own rows and every row they point to (the union, gathered
// on the host), read through an id -> compact-row map (ROWS 1), so each row
// counts its detours exactly as in the resident prune.
static void prune_chunked(Ctx& c, const uint32_t* san, int64_t N, int M, int K, size_t budget, uint32_t* out,
                          OocReport* rep)
{
    GT_REQUIRE(K >= 1 && K <= M && M <= 128, "bad degrees");
    const size_t fixed = static_cast<size_t>(N) * sizeof(int32_t);   // the id map
    // per chunk row, at worst: its own row and M neighbour rows, list entries, the output row
    const size_t per_row = static_cast<size_t>(M + 1) * (static_cast<size_t>(M) * 4 + 4) + static_cast<size_t>(K) * 4;
    GT_REQUIRE(budget > fixed + 64 * per_row, "device budget too small for the chunked prune (need > " +
                                                  std::to_string((fixed + 64 * per_row) >> 20) + " MiB)");
    const int64_t chunk = std::min<int64_t>(N, static_cast<int64_t>((budget - fixed) / per_row));
    int32_t* cidx = c.ws<int32_t>(W_OOC_A, static_cast<size_t>(N));
    const size_t umax = static_cast<size_t>(chunk) * (M + 1);
    uint32_t* Gc = c.ws<uint32_t>(W_OOC_B, umax * M);
    int32_t* ulist = c.ws<int32_t>(W_OOC_C, umax);
    uint32_t* dout = c.ws<uint32_t>(W_OOC_D, static_cast<size_t>(chunk) * K);
    unsigned long long* bad = c.ws<unsigned long long>(W_FLAG, 1);
    int* err = c.ws<int>(W_TMP, 1);
    launch_init_flags(bad, err, c.s);
    HostBuf hrows, hlist, hout;
    uint32_t* st_rows = hrows.as<uint32_t>(umax * M);
    int32_t* st_list = hlist.as<int32_t>(umax);
    uint32_t* st_out = hout.as<uint32_t>(static_cast<size_t>(chunk) * K);
    std::vector<int32_t> mark(static_cast<size_t>(N), -1);
    int32_t gen = 0;
    for (int64_t a0 = 0; a0 < N; a0 += chunk, ++gen) {
        const int64_t n = std::min(chunk, N - a0);
        // the union: the chunk's rows, then the rows they point to
        size_t nu = 0;
        for (int64_t i = a0; i < a0 + n; ++i) {
            mark[static_cast<size_t>(i)] = gen;
            st_list[nu++] = static_cast<int32_t>(i);
        }
        for (int64_t i = a0; i < a0 + n; ++i)
            for (int k = 0; k < M; ++k) {
                const uint32_t d = san[i * M + k];
                if (d < N && mark[d] != gen) {
                    mark[d] = gen;
                    st_list[nu++] = static_cast<int32_t>(d);
                }
            }
        parallel_slices(static_cast<int64_t>(nu), host_threads(), [&](int, int64_t lo, int64_t hi) {
            for (int64_t u = lo; u < hi; ++u)
                std::memcpy(st_rows + u * M, san + static_cast<int64_t>(st_list[u]) * M, static_cast<size_t>(M) * 4);
        });
        c.h2d(Gc, st_rows, nu * M * sizeof(uint32_t));
        c.h2d(ulist, st_list, nu * sizeof(int32_t));
        launch_set_cidx(ulist, static_cast<int64_t>(nu), cidx, c.s);
        PruneMap map{};
        map.a0 = a0;
        map.n = n;
        map.cidx = cidx;
        launch_cagra_prune_mapped(reinterpret_cast<const int32_t*>(Gc), N, M, K, dout, bad, map, 1, c.s);
        c.d2h(st_out, dout, static_cast<size_t>(n) * K * sizeof(uint32_t));
        c.sync();   // the staging buffers are refilled by the next chunk
        std::memcpy(out + a0 * K, st_out, static_cast<size_t>(n) * K * sizeof(uint32_t));
        if (rep) {
            rep->chunks++;
            rep->rows_moved += static_cast<double>(nu);
        }
    }
    unsigned long long h = 0;
    c.d2h(&h, bad, sizeof(h));
    c.sync();
    if (h != ~0ull)
        throw Error(GT_EFEWCAND, "prune: row " + std::to_string(h) + " has fewer than output_degree valid candidates");
}

// Multi-chunk reverse merge (Method E, src/optimize_chunked.cu:1548-2057) of a
// host forward graph fwd (N x K) into host rows out.  Phase 1 streams the
// forward rows in batches through the device, which routes every edge to its
// destination chunk as a (rank, row in chunk, source) record; the host keeps
// each chunk's records.  Phase 2 takes one destination chunk at a time:
// records and forward rows up, records grouped per row (CSR), rows merged by
// rev_merge_kernel -- the same rows as gt_reverse_merge.
static void reverse_merge_chunked(Ctx& c, const uint32_t* fwd, int64_t N, int K, size_t budget, uint32_t* out,
                                  OocReport* rep)
{
    GT_REQUIRE(K >= 1 && K <= 64, "output degree must be in [1, 64]");
    // phase 2 per destination row: forward and output rows, about K records
    // (record, key, slot), row count and offset
    const size_t per_row2 = static_cast<size_t>(K) * (8 + 20) + 12;
    const size_t per_row1 = static_cast<size_t>(K) * (4 + 8);   // phase 1: a forward row and its records
    GT_REQUIRE(budget >= 64 * std::max(per_row1, per_row2), "device budget too small for the chunked merge");
    int64_t R = std::min<int64_t>(N, std::min<int64_t>(int64_t(1) << 26, static_cast<int64_t>(budget / per_row2)));
    const int64_t nchunks = ceil_div(N, R);
    GT_REQUIRE(nchunks <= 4096, "device budget too small for the chunked merge (more than 4096 chunks)");
    const int64_t B = std::min<int64_t>(N, static_cast<int64_t>(budget / per_row1));
    uint32_t* dfwd = c.ws<uint32_t>(W_OOC_A, static_cast<size_t>(B) * K);
    unsigned long long* drec = c.ws<unsigned long long>(W_OOC_B, static_cast<size_t>(B) * K);
    uint32_t* counts = c.ws<uint32_t>(W_OOC_C, static_cast<size_t>(2 * nchunks));
    uint32_t* cursor = counts + nchunks;
    int* err = c.ws<int>(W_TMP, 1);
    unsigned long long* bad = c.ws<unsigned long long>(W_FLAG, 1);
    launch_init_flags(bad, err, c.s);
    std::vector<std::vector<uint64_t>> recs(static_cast<size_t>(nchunks));
    std::vector<uint32_t> h_counts(static_cast<size_t>(nchunks)), h_off(static_cast<size_t>(nchunks));
    HostBuf hrec;
    uint64_t* st_rec = hrec.as<uint64_t>(static_cast<size_t>(B) * K);
    for (int64_t s0 = 0; s0 < N; s0 += B) {
        const int64_t nb = std::min(B, N - s0);
        c.h2d(dfwd, fwd + s0 * K, static_cast<size_t>(nb) * K * sizeof(uint32_t));
        GT_HIP(hipMemsetAsync(counts, 0, static_cast<size_t>(nchunks) * sizeof(uint32_t), c.s));
        launch_route(dfwd, nb, K, N, R, static_cast<int>(nchunks), s0, counts, cursor, drec, err, false, c.s);
        c.d2h(h_counts.data(), counts, h_counts.size() * sizeof(uint32_t));
        c.sync();
        uint32_t tot = 0;
        for (int64_t q = 0; q < nchunks; ++q) {
            h_off[static_cast<size_t>(q)] = tot;
            tot += h_counts[static_cast<size_t>(q)];
        }
        c.h2d(cursor, h_off.data(), h_off.size() * sizeof(uint32_t));
        launch_route(dfwd, nb, K, N, R, static_cast<int>(nchunks), s0, counts, cursor, drec, err, true, c.s);
        c.d2h(st_rec, drec, static_cast<size_t>(tot) * sizeof(uint64_t));
        c.sync();
        for (int64_t q = 0; q < nchunks; ++q) {
            std::vector<uint64_t>& v = recs[static_cast<size_t>(q)];
            const uint64_t* src = st_rec + h_off[static_cast<size_t>(q)];
            v.insert(v.end(), src, src + h_counts[static_cast<size_t>(q)]);
        }
    }
    int h_err = 0;
    c.d2h(&h_err, err, sizeof(int));
    c.sync();
    if (h_err) throw Error(GT_EINVAL, "reverse merge: forward graph holds an id >= N");
    HostBuf hout;
    uint32_t* st_out = hout.as<uint32_t>(static_cast<size_t>(R) * K);
    // phase 2 on destination rows [c0, c0 + nr) and their records v (row
    // local to c0)
    auto merge_rows = [&](int64_t c0, int64_t nr, const std::vector<uint64_t>& v) {
        const int64_t nrec = static_cast<int64_t>(v.size());
        unsigned long long* d_rec = c.ws<unsigned long long>(W_OOC_B, static_cast<size_t>(std::max<int64_t>(nrec, 1)));
        unsigned long long* d_key = c.ws<unsigned long long>(W_OOC_E, static_cast<size_t>(std::max<int64_t>(nrec, 1)));
        uint32_t* d_slot = c.ws<uint32_t>(W_OOC_F, static_cast<size_t>(std::max<int64_t>(nrec, 1)));
        uint32_t* d_deg = c.ws<uint32_t>(W_DEG, static_cast<size_t>(nr));
        uint32_t* d_off = c.ws<uint32_t>(W_OFF, static_cast<size_t>(nr) + 1);
        uint32_t* d_sums = c.ws<uint32_t>(W_SUMS, static_cast<size_t>(ceil_div(nr, 1024) + 1));
        uint32_t* d_fwd = c.ws<uint32_t>(W_OOC_A, static_cast<size_t>(nr) * K);
        uint32_t* d_out = c.ws<uint32_t>(W_OOC_G, static_cast<size_t>(nr) * K);
        c.h2d(d_rec, v.data(), static_cast<size_t>(nrec) * sizeof(uint64_t));
        c.h2d(d_fwd, fwd + c0 * K, static_cast<size_t>(nr) * K * sizeof(uint32_t));
        GT_HIP(hipMemsetAsync(d_deg, 0, static_cast<size_t>(nr) * sizeof(uint32_t), c.s));
        launch_rec_group(d_rec, nrec, d_deg, d_slot, nullptr, nullptr, false, c.s);
        launch_exclusive_scan(d_deg, nr, d_off, d_sums, c.s);
        launch_rec_group(d_rec, nrec, nullptr, d_slot, d_off, d_key, true, c.s);
        launch_rev_merge(d_fwd, nr, K, d_off, d_key, d_out, c.s);
        c.d2h(st_out, d_out, static_cast<size_t>(nr) * K * sizeof(uint32_t));
        c.sync();
        std::memcpy(out + c0 * K, st_out, static_cast<size_t>(nr) * K * sizeof(uint32_t));
        if (rep) {
            rep->chunks++;
            rep->rows_moved += static_cast<double>(nr);
        }
    };
    // A chunk holds about R * K records (one per forward edge into it), which
    // the budget was sized for; a chunk whose rows receive more (hub rows) is
    // merged in row ranges whose records fit, a single row over that alone.
    const size_t cap = static_cast<size_t>(R) * K;
    constexpr uint64_t kLocal = 0x3FFFFFFull;   // a record's row within its chunk: bits 32..57
    for (int64_t q = 0; q < nchunks; ++q) {
        const int64_t c0 = q * R, nr = std::min(R, N - c0);
        const std::vector<uint64_t>& v = recs[static_cast<size_t>(q)];
        if (v.size() <= cap) {
            merge_rows(c0, nr, v);
            continue;
        }
        std::vector<size_t> cnt(static_cast<size_t>(nr), 0);
        for (const uint64_t r : v) cnt[static_cast<size_t>((r >> 32) & kLocal)]++;
        for (int64_t a = 0; a < nr;) {
            int64_t b = a + 1;
            size_t sum = cnt[static_cast<size_t>(a)];
            while (b < nr && sum + cnt[static_cast<size_t>(b)] <= cap) sum += cnt[static_cast<size_t>(b++)];
            std::vector<uint64_t> sub;
            sub.reserve(sum);
            for (const uint64_t r : v) {
                const int64_t dl = static_cast<int64_t>((r >> 32) & kLocal);
                if (dl >= a && dl < b) sub.push_back(r - (static_cast<uint64_t>(a) << 32));
            }
            merge_rows(c0 + a, b - a, sub);
            a = b;
        }
    }
}

// prune_windowed_gpu::run_chunked (src/prune_windowed_gpu.cu:529-915) with
// the candidates ranked as given (its --dists ranking of sorted rows):
// bucket position q owns the ids [off[q], off[q + 1]); row a at position p
// counts a detour through its neighbour d only when d's position is in p's
// window (win[p * W ..], win_len[p] entries), otherwise d contributes
// nothing (src/prune_windowed_core.hpp:177-232).  Positions go in chunks
// whose window union -- every row of every bucket in the windows -- fits the
// budget; a chunk's buckets sit in a compact device table (ROWS 2), so the
// rows do not depend on the chunking.
static void prune_windowed_chunked(Ctx& c, const int32_t* cand, int64_t N, int M, const uint32_t* off, int nb,
                                   const int32_t* win, const int32_t* win_len, int W, int K, size_t budget,
                                   uint32_t* out, OocReport* rep)
{
    GT_REQUIRE(K >= 1 && K <= M && M <= 128, "bad degrees");
    GT_REQUIRE(nb >= 1 && off[0] == 0 && static_cast<int64_t>(off[nb]) == N, "bucket offsets must cover [0, N)");
    for (int q = 0; q < nb; ++q) GT_REQUIRE(off[q] <= off[q + 1], "bucket offsets must be ascending");
    for (int q = 0; q < nb; ++q) {
        GT_REQUIRE(win_len[q] >= 0 && win_len[q] <= W, "window length out of range");
        for (int i = 0; i < win_len[q]; ++i)
            GT_REQUIRE(win[static_cast<int64_t>(q) * W + i] >= 0 && win[static_cast<int64_t>(q) * W + i] < nb,
                       "window position out of range");
    }
    const size_t row_bytes = static_cast<size_t>(M) * 4;
    const size_t fixed = static_cast<size_t>(nb) * (8 + 4 + 4) + static_cast<size_t>(nb) * W * 4;
    GT_REQUIRE(budget > fixed, "device budget too small for the windowed prune");
    const int64_t cap_rows = static_cast<int64_t>((budget - fixed) / (row_bytes + static_cast<size_t>(K) * 4));
    uint32_t* d_off = c.ws<uint32_t>(W_OOC_C, static_cast<size_t>(nb) + 1);
    int32_t* d_win = c.ws<int32_t>(W_OOC_D, static_cast<size_t>(nb) * W + 1);
    int32_t* d_wl = c.ws<int32_t>(W_OOC_E, static_cast<size_t>(nb));
    int64_t* d_cbase = c.ws<int64_t>(W_OOC_F, static_cast<size_t>(nb));
    c.h2d(d_off, off, (static_cast<size_t>(nb) + 1) * sizeof(uint32_t));
    c.h2d(d_win, win, static_cast<size_t>(nb) * W * sizeof(int32_t));
    c.h2d(d_wl, win_len, static_cast<size_t>(nb) * sizeof(int32_t));
    unsigned long long* bad = c.ws<unsigned long long>(W_FLAG, 1);
    int* err = c.ws<int>(W_TMP, 1);
    launch_init_flags(bad, err, c.s);
    std::vector<int32_t> stamp(static_cast<size_t>(nb), -1);
    std::vector<int64_t> cbase(static_cast<size_t>(nb));
    std::vector<int32_t> U;
    HostBuf hrows, hout;
    int32_t chunk_id = 0;
    for (int p0 = 0; p0 < nb; ++chunk_id) {
        // the longest run of positions from p0 whose window union fits
        // (always at least one position, which must fit by itself)
        U.clear();
        int64_t rows = 0;
        int p1 = p0;
        auto add = [&](int q) {
            if (stamp[static_cast<size_t>(q)] == chunk_id) return;
            stamp[static_cast<size_t>(q)] = chunk_id;
            U.push_back(q);
            rows += static_cast<int64_t>(off[q + 1] - off[q]);
        };
        while (p1 < nb) {
            const size_t u0 = U.size();
            const int64_t r0 = rows;
            add(p1);
            for (int i = 0; i < win_len[p1]; ++i) add(win[static_cast<int64_t>(p1) * W + i]);
            if (p1 > p0 && rows > cap_rows) {   // undo: p1 starts the next chunk
                for (size_t i = u0; i < U.size(); ++i) stamp[static_cast<size_t>(U[i])] = -1;
                U.resize(u0);
                rows = r0;
                break;
            }
            ++p1;
        }
        GT_REQUIRE(rows <= cap_rows || p1 == p0 + 1,
                   "device budget too small for the windowed prune (one window needs more)");
        std::fill(cbase.begin(), cbase.end(), int64_t(-1));
        int64_t at = 0;
        for (int q : U) {
            cbase[static_cast<size_t>(q)] = at;
            at += static_cast<int64_t>(off[q + 1] - off[q]);
        }
        int32_t* st_rows = hrows.as<int32_t>(static_cast<size_t>(std::max<int64_t>(at, 1)) * M);
        parallel_slices(static_cast<int64_t>(U.size()), host_threads(), [&](int, int64_t lo, int64_t hi) {
            for (int64_t i = lo; i < hi; ++i) {
                const int q = U[static_cast<size_t>(i)];
                std::memcpy(st_rows + cbase[static_cast<size_t>(q)] * M, cand + static_cast<int64_t>(off[q]) * M,
                            static_cast<size_t>(off[q + 1] - off[q]) * row_bytes);
            }
        });
        int32_t* Gc = c.ws<int32_t>(W_OOC_B, static_cast<size_t>(std::max<int64_t>(at, 1)) * M);
        const int64_t a0 = off[p0], n = static_cast<int64_t>(off[p1]) - a0;
        uint32_t* dout = c.ws<uint32_t>(W_OOC_G, static_cast<size_t>(std::max<int64_t>(n, 1)) * K);
        c.h2d(Gc, st_rows, static_cast<size_t>(at) * row_bytes);
        c.h2d(d_cbase, cbase.data(), cbase.size() * sizeof(int64_t));
        PruneMap map{};
        map.a0 = a0;
        map.n = n;
        map.off = d_off;
        map.win = d_win;
        map.win_len = d_wl;
        map.cbase = d_cbase;
        map.n_buckets = nb;
        map.W = W;
        launch_cagra_prune_mapped(Gc, N, M, K, dout, bad, map, 2, c.s);
        uint32_t* st_out = hout.as<uint32_t>(static_cast<size_t>(std::max<int64_t>(n, 1)) * K);
        c.d2h(st_out, dout, static_cast<size_t>(n) * K * sizeof(uint32_t));
        c.sync();   // staging and cbase are refilled by the next chunk
        std::memcpy(out + a0 * K, st_out, static_cast<size_t>(n) * K * sizeof(uint32_t));
        if (rep) {
            rep->chunks++;
            rep->rows_moved += static_cast<double>(at);
        }
        p0 = p1;
    }
    unsigned long long h = 0;
    c.d2h(&h, bad, sizeof(h));
    c.sync();
    if (h != ~0ull)
        throw Error(GT_EFEWCAND, "prune: row " + std::to_string(h) + " has fewer than output_degree valid candidates");
}

// One round of the out-of-core build (src/bucket.cu:5670-6369: the running
// table in host memory, merged chunk by chunk): buckets in order, grouped
// into chunks whose members fit the budget (a bucket is the smallest unit).
// A chunk's members' running rows go up (round > 0), its buckets' lists are
// computed into compact rows (seeded from the running rows) and merged with
// them on the device, and the merged rows go back into the host table.  Every
// row gets the lists and merges of the resident build, so the table is the
// same.
static void ooc_round(Ctx& c, const DevMatrix& X, const Buckets& b, int M, int metric, int r, int32_t* h_ids,
                      float* h_d, size_t budget, gt_build_stats& st, OocReport* rep)
{
    const int64_t C = static_cast<int64_t>(b.offsets.size()) - 1;
    // per member row: running, new and merged lists, the collect launch's candidates
    const size_t per_row = static_cast<size_t>(M) * 8 * 4 + static_cast<size_t>(kCollectCap) * 8 + 8;
    const int64_t cap = std::max<int64_t>(kQueriesPerBlock, static_cast<int64_t>(budget / per_row));
    HostBuf hi, hd;
    for (int64_t b0 = 0; b0 < C;) {
        int64_t b1 = b0, rows = 0;
        while (b1 < C) {
            const int64_t nb = b.offsets[static_cast<size_t>(b1 + 1)] - b.offsets[static_cast<size_t>(b1)];
            if (b1 > b0 && rows + nb > cap) break;
            rows += nb;
            ++b1;
        }
        const int64_t q0 = b.offsets[static_cast<size_t>(b0)];
        const size_t nm = static_cast<size_t>(std::max<int64_t>(rows, 1)) * M;
        int32_t* rid = c.ws<int32_t>(W_G1, nm);
        float* rdd = c.ws<float>(W_G2, nm);
        int32_t* nid = c.ws<int32_t>(W_IDS, nm);
        float* ndd = c.ws<float>(W_D, nm);
        int32_t* mid = c.ws<int32_t>(W_IDS2, nm);
        float* mdd = c.ws<float>(W_D2, nm);
        int32_t* sti = hi.as<int32_t>(nm);
        float* std_ = hd.as<float>(nm);
        const int32_t* mem = b.members.data() + q0;
        if (r > 0) {
            parallel_slices(rows, host_threads(), [&](int, int64_t lo, int64_t hi_) {
                for (int64_t q = lo; q < hi_; ++q) {
                    std::memcpy(sti + q * M, h_ids + static_cast<int64_t>(mem[q]) * M, static_cast<size_t>(M) * 4);
                    std::memcpy(std_ + q * M, h_d + static_cast<int64_t>(mem[q]) * M, static_cast<size_t>(M) * 4);
                }
            });
            c.h2d(rid, sti, static_cast<size_t>(rows) * M * 4);
            c.h2d(rdd, std_, static_cast<size_t>(rows) * M * 4);
        }
        int32_t* oi = mid;
        float* od = mdd;
        // a pass seeded with the running rows (rid, rdd), merged into them in
        // place by the collect launch, else through (nid, ndd) into (mid, mdd)
        auto seeded = [&](bool own, bool probes) {
            bool merged = false;
            st.t_knn += bucketed_round(c, X, b, M, metric, rdd, nid, ndd, &st.max_pool, &st.max_bucket,
                                       &st.knn_pairs, own, probes, b0, b1, rid, &merged);
            if (merged) {
                oi = rid;
                od = rdd;
            } else {
                st.t_merge += c.timed([&] { launch_merge_rounds(rid, rdd, nid, ndd, rows, M, mid, mdd, c.s); });
            }
        };
        if (r == 0 && b.P > 0) {
            // own buckets unseeded, then the probe buckets seeded with their M-th distance, merged
            st.t_knn += bucketed_round(c, X, b, M, metric, nullptr, rid, rdd, &st.max_pool, &st.max_bucket,
                                       &st.knn_pairs, true, false, b0, b1);
            seeded(false, true);
        } else if (r == 0) {
            st.t_knn += bucketed_round(c, X, b, M, metric, nullptr, mid, mdd, &st.max_pool, &st.max_bucket,
                                       &st.knn_pairs, true, true, b0, b1);
        } else {
            seeded(true, true);
        }
        c.d2h(sti, oi, static_cast<size_t>(rows) * M * 4);
        c.d2h(std_, od, static_cast<size_t>(rows) * M * 4);
        c.sync();
        parallel_slices(rows, host_threads(), [&](int, int64_t lo, int64_t hi_) {
            for (int64_t q = lo; q < hi_; ++q) {
                std::memcpy(h_ids + static_cast<int64_t>(mem[q]) * M, sti + q * M, static_cast<size_t>(M) * 4);
                std::memcpy(h_d + static_cast<int64_t>(mem[q]) * M, std_ + q * M, static_cast<size_t>(M) * 4);
            }
        });
        if (rep) {
            rep->chunks++;
            rep->rows_moved += static_cast<double>(rows);
        }
        b0 = b1;
    }
}

}  // namespace gtann

using namespace gtann;

// ---------------------------------------------------------------- fixed scratch of gt_optimize_noalloc
// One array per GPU, allocated with the code object and held until the
// process ends.  Host code never uses the name `scratch` as an address (on
// the host it only stands for the symbol): gt_create looks up each device's
// own address with hipGetSymbolAddress, once per device, and every use goes
// through that pointer.
static __device__ __align__(256) unsigned char scratch[GT_NOALLOC_SCRATCH_BYTES];

namespace {
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};
std::string g_scratch_err[kMaxDevices];

// with `device` current
void* scratch_for_device(int device, std::string& why)
{
    if (device < 0 || device >= kMaxDevices) {
        why = "device index beyond the scratch table";
        return nullptr;
    }
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    if (!g_scratch_ptr[device] && g_scratch_err[device].empty()) {
        void* p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !p) {
            g_scratch_err[device] = std::string("hipGetSymbolAddress(scratch): ") + hipGetErrorString(e);
            (void)hipGetLastError();
        } else {
            g_scratch_ptr[device] = p;
        }
    }
    why = g_scratch_err[device];
    return g_scratch_ptr[device];
}

// Byte offsets of gt_optimize_noalloc's buffers inside the scratch array
// (each 256-byte aligned): the forward graph, the two flags, and the binned
// reverse merge's histogram, offsets, scan sums, partitioned and grouped keys.
struct NoAllocLayout {
    size_t fwd, bad, err, hist, offs, sums, part, grouped, bytes;
};

NoAllocLayout noalloc_layout(int64_t N, int K)
{
    const int64_t E = N * K;
    const int shift = rev_bin_shift(N);
    const int64_t nh = ceil_div(N, int64_t(1) << shift) * rev_bin_blocks(E);
    auto up = [](size_t x) { return (x + 255) / 256 * 256; };
    NoAllocLayout L{};
    size_t o = 0;
    L.fwd = o;     o += up(static_cast<size_t>(E) * sizeof(uint32_t));
    L.bad = o;     o += up(sizeof(unsigned long long));
    L.err = o;     o += up(sizeof(int));
    L.hist = o;    o += up(static_cast<size_t>(nh) * sizeof(uint32_t));
    L.offs = o;    o += up(static_cast<size_t>(nh + 1) * sizeof(uint32_t));
    L.sums = o;    o += up(static_cast<size_t>(ceil_div(nh, 1024) + 1) * sizeof(uint32_t));
    L.part = o;    o += up(static_cast<size_t>(E) * sizeof(unsigned long long));
    L.grouped = o; o += up(static_cast<size_t>(E) * sizeof(unsigned long long));
    L.bytes = o;
    return L;
}

bool on_device(const void* p, int device)
{
    if (!p) return false;
    hipPointerAttribute_t attr;
    if (hipPointerGetAttributes(&attr, p) != hipSuccess) {
        (void)hipGetLastError();
        return false;
    }
    return attr.type == hipMemoryTypeDevice && attr.device == device;
}
}  // namespace

template <typename F>
static int guarded(gt_ctx* ctx, F&& f)
{
    if (!ctx) return GT_EINVAL;
    try {
        GT_HIP(hipSetDevice(ctx->device));
        ctx->err.clear();
        f();
        return GT_OK;
    } catch (const Error& e) {
        ctx->err = e.what();
        (void)hipStreamSynchronize(ctx->stream);
        return e.code;
    } catch (const std::exception& e) {
        ctx->err = e.what();
        return GT_EINVAL;
    } catch (...) {
        ctx->err = "unknown error";
        return GT_EINVAL;
    }
}

// Host-only entry points (bucket order / reorder) also run without a
// context on host buffers; their errors then go to this thread's message,
// which gt_last_error(NULL) returns.
thread_local std::string g_host_err;

template <typename F>
static int guarded_host(gt_ctx* ctx, F&& f)
{
    if (ctx) return guarded(ctx, [&] { f(ctx); });
    try {
        g_host_err.clear();
        f(nullptr);
        return GT_OK;
    } catch (const Error& e) {
        g_host_err = e.what();
        return e.code;
    } catch (const std::exception& e) {
        g_host_err = e.what();
        return GT_EINVAL;
    }
}

// copies between a caller buffer (host, or device when ctx is given) and host memory
template <typename T>
static void fetch_host(gt_ctx* ctx, T* dst, const T* src, size_t n)
{
    if (!n) return;
    if (ctx && is_device_ptr(src)) {
        Ctx c(ctx);
        c.d2h(dst, src, n * sizeof(T));
        c.sync();
    } else {
        std::memcpy(dst, src, n * sizeof(T));
    }
}
template <typename T>
static void store_host(gt_ctx* ctx, T* dst, const T* src, size_t n)
{
    if (!n) return;
    if (ctx && is_device_ptr(dst)) {
        Ctx c(ctx);
        c.h2d(dst, src, n * sizeof(T));
        c.sync();
    } else {
        std::memcpy(dst, src, n * sizeof(T));
    }
}

extern "C" {

const char* gt_version(void) { return "gtann-gfx950 0.1"; }

int gt_create(int device, gt_ctx** out)
{
    if (!out) return GT_EINVAL;
    *out = nullptr;
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || device < 0 || device >= n) return GT_EDEVICE;
    gt_ctx* c = new (std::nothrow) gt_ctx();
    if (!c) return GT_ENOMEM;
    c->device = device;
    gt_debug_opts_default(&c->dbg);
    // A blocking stream: every call's work is ordered after work already
    // queued on the device's legacy null stream (PyTorch's default stream),
    // so a device buffer produced there asynchronously is complete before
    // the library reads it.
    if (hipSetDevice(device) != hipSuccess || hipStreamCreateWithFlags(&c->stream, hipStreamDefault) != hipSuccess ||
        hipEventCreate(&c->ev0) != hipSuccess || hipEventCreate(&c->ev1) != hipSuccess ||
        hipEventCreate(&c->members_up[0]) != hipSuccess || hipEventCreate(&c->members_up[1]) != hipSuccess) {
        delete c;
        return GT_EDEVICE;
    }
    // this device's scratch address (looked up once per device); a failure
    // only disables gt_optimize_noalloc
    c->scratch = scratch_for_device(device, c->scratch_err);
    *out = c;
    return GT_OK;
}

void gt_destroy(gt_ctx* ctx)
{
    if (!ctx) return;
    (void)hipSetDevice(ctx->device);
    (void)hipStreamSynchronize(ctx->stream);
    for (auto& b : ctx->ws) {
        if (b.p) (void)hipFree(b.p);
        b.p = nullptr;
        b.cap = 0;
    }
    for (auto& pb : ctx->pinned) pb.release();
    ctx->pin_lloyd.release();
    for (gtann::HostBuf& b : ctx->pin_bucket) b.release();
    if (ctx->ev0) (void)hipEventDestroy(ctx->ev0);
    if (ctx->ev1) (void)hipEventDestroy(ctx->ev1);
    for (hipEvent_t e : ctx->members_up)
        if (e) (void)hipEventDestroy(e);
    if (ctx->stream) (void)hipStreamDestroy(ctx->stream);
    delete ctx;
}

const char* gt_last_error(const gt_ctx* ctx)
{
    if (ctx) return ctx->err.c_str();
    return g_host_err.empty() ? "null context" : g_host_err.c_str();
}

void gt_build_params_default(gt_build_params* p)
{
    if (!p) return;
    p->metric = GT_METRIC_L2;
    p->n_buckets = 0;   // 0 = N / 4000
    p->nprobe = 1;      // -1 = the reference's rule ceil(20000 / avg bucket) (sk/scripts/dataset_env.py:12,56)
    p->M = 64;
    p->K = 32;
    p->rounds = 2;
    p->refine_passes = 0;
    p->refine_sample = 16;
    p->kmeans_iters = 3;
    p->balance = 0.8f;
    p->seed = 42;
    p->reverse_edges = 0;
    p->int_exact = 1;
    p->device_budget_mb = 0;
    p->seeding = GT_SEED_AUTO;
    p->kmeans_train_fraction = 0.f;
}

void gt_debug_opts_default(gt_debug_opts* o)
{
    if (!o) return;
    *o = gt_debug_opts{};
    o->knn_collect = 1;
    o->revmerge_path = 0;
    o->sub_order = 1;
    o->lloyd_host_csr = 0;
    o->prune_flat_rows = 0;
    o->knn_stats = 0;
    o->knn_prune = 1;
    o->knn_resident = 1;
    o->knn_screen = 1;
}

int gt_set_debug(gt_ctx* ctx, const gt_debug_opts* o)
{
    if (!ctx) return GT_EINVAL;
    gt_debug_opts d;
    gt_debug_opts_default(&d);
    if (o) d = *o;
    if (d.knn_window < 0 || d.knn_window > 32 || (d.knn_window & 1)) {
        ctx->err = "gt_set_debug: knn_window must be 0 or an even number of tiles up to 32";
        return GT_EINVAL;
    }
    if (d.revmerge_path < 0 || d.revmerge_path > 4) {
        ctx->err = "gt_set_debug: revmerge_path must be 0..4";
        return GT_EINVAL;
    }
    ctx->dbg = d;
    return GT_OK;
}

int gt_reverse_merge_chunked(gt_ctx* ctx, const uint32_t* fwd, int64_t N, int32_t K, int64_t device_budget_bytes,
                             uint32_t* out)
{
    return guarded(ctx, [&] {
        GT_REQUIRE(fwd && out && N >= 1 && K >= 1 && K <= 64, "bad arguments");
        GT_REQUIRE(!is_device_ptr(fwd) && !is_device_ptr(out), "gt_reverse_merge_chunked takes host buffers");
        Ctx c(ctx);
        const size_t budget = device_budget_bytes > 0 ? static_cast<size_t>(device_budget_bytes)
                                                      : static_cast<size_t>(N) * K * 64 + (size_t(64) << 20);
        reverse_merge_chunked(c, fwd, N, K, budget, out, nullptr);
    });
}

int gt_prune_windowed(gt_ctx* ctx, const int32_t* cand, int64_t N, int32_t M, const uint32_t* offsets,
                      int32_t n_buckets, const int32_t* win, const int32_t* win_len, int32_t W, int32_t K,
                      int64_t device_budget_bytes, uint32_t* out)
{
    return guarded(ctx, [&] {
        GT_REQUIRE(cand && offsets && win && win_len && out && N >= 1 && M >= 1 && n_buckets >= 1 && W >= 1,
                   "bad arguments");
        GT_REQUIRE(N < (int64_t(1) << 31), "N must be < 2^31");
        GT_REQUIRE(!is_device_ptr(cand) && !is_device_ptr(out), "gt_prune_windowed takes host buffers");
        Ctx c(ctx);
        const size_t budget = device_budget_bytes > 0
                                  ? static_cast<size_t>(device_budget_bytes)
                                  : static_cast<size_t>(N) * (M + K) * 4 + static_cast<size_t>(n_buckets) * (W + 8) * 4 +
                                        (size_t(1) << 20);
        prune_windowed_chunked(c, cand, N, M, offsets, n_buckets, win, win_len, W, K, budget, out, nullptr);
    });
}

void gt_search_params_default(gt_search_params* p)
{
    if (!p) return;
    p->topk = 10;
    p->ef = 200;
    p->num_entry = 4;
    p->metric = GT_METRIC_L2;
    p->seed = 42;
    p->visited_slots = 0;
    p->reserved_ = 0;
}

int gt_search(gt_ctx* ctx, const void* X, int64_t N, int32_t D, int dtype, const uint32_t* graph, int32_t degree,
              const void* Q, int64_t nq, const int32_t* entries, int32_t n_entry, const gt_search_params* params,
              int32_t* out_ids, float* out_d, gt_search_stats* stats)
{
    return guarded(ctx, [&] {
        GT_REQUIRE(params && graph && out_ids && out_d && nq >= 0, "bad arguments");
        const gt_search_params& p = *params;
        GT_REQUIRE(degree >= 1, "degree must be >= 1");
        GT_REQUIRE(p.topk >= 1 && p.topk <= 2048, "topk must be in [1, 2048]");
        const int ef = std::max(p.ef, p.topk);
        GT_REQUIRE(ef <= 2048, "ef must be <= 2048");
        GT_REQUIRE(p.metric == GT_METRIC_L2 || p.metric == GT_METRIC_IP, "unknown metric");
        GT_REQUIRE(N < (int64_t(1) << 31) - 1, "N must be < 2^31 - 1");
        Timer tt;
        Ctx c(ctx);
        DevMatrix Xm = prepare(c, W_X, W_XRAW, W_NORMS, X, N, D, dtype);
        gt_search_stats st{};
        if (nq > 0) {
            GT_REQUIRE(Q != nullptr, "no queries");
            DevMatrix Qm = prepare(c, W_C, W_CRAW, W_CNORMS, Q, nq, D, dtype);
            const uint32_t* g = c.in<uint32_t>(W_IN, graph, static_cast<size_t>(N) * degree);
            int E = n_entry;
            const int32_t* d_ent = nullptr;
            if (entries) {
                GT_REQUIRE(n_entry >= 1 && n_entry <= 64, "1 <= n_entry <= 64");
                d_ent = c.in<int32_t>(W_PROBE_I, entries, static_cast<size_t>(nq) * E);
            } else {
                E = p.num_entry;
                GT_REQUIRE(E >= 1 && E <= 64, "1 <= num_entry <= 64");
                // E draws per query from a splitmix64 stream, sorted and distinct
                std::vector<int32_t> he(static_cast<size_t>(nq) * E, -1);
                parallel_slices(nq, host_threads(), [&](int, int64_t lo, int64_t hi) {
                    std::vector<int32_t> tmp(static_cast<size_t>(E));
                    for (int64_t q = lo; q < hi; ++q) {
                        for (int e = 0; e < E; ++e) {
                            uint64_t z = p.seed + 0x9E3779B97F4A7C15ull * static_cast<uint64_t>(q * E + e + 1);
                            z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
                            z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
                            z ^= z >> 31;
                            tmp[static_cast<size_t>(e)] = static_cast<int32_t>(z % static_cast<uint64_t>(N));
                        }
                        std::sort(tmp.begin(), tmp.end());
                        const auto end = std::unique(tmp.begin(), tmp.end());
                        std::copy(tmp.begin(), end, he.begin() + q * E);
                    }
                });
                int32_t* d = c.ws<int32_t>(W_PROBE_I, he.size());
                c.h2d(d, he.data(), he.size() * sizeof(int32_t));
                c.sync();   // he is released at the end of this scope
                d_ent = d;
            }
            const size_t nr = static_cast<size_t>(nq) * p.topk;
            int32_t* oi = c.in<int32_t>(W_IDS, out_ids, nr, false);
            float* od = c.in<float>(W_D, out_d, nr, false);
            int32_t* d_status = c.ws<int32_t>(W_FLAG, static_cast<size_t>(nq));
            int32_t* d_exp = c.ws<int32_t>(W_DEG, static_cast<size_t>(nq));
            int32_t* d_vis = c.ws<int32_t>(W_CUR, static_cast<size_t>(nq));

            SearchArgs a{};
            a.X = Xm.data;
            a.N = N;
            a.D = D;
            a.Dp = Xm.Dp;
            a.graph = g;
            a.deg = degree;
            a.Q = Qm.data;
            a.entries = d_ent;
            a.n_entry = E;
            a.n_run = nq;
            a.topk = p.topk;
            a.ef = ef;
            a.metric = p.metric;
            a.efr = static_cast<int32_t>(ceil_div(ef, 64) * 64);
            a.CC = a.efr + 256;
            a.out_ids = oi;
            a.out_d = od;
            a.status = d_status;
            a.expansions = d_exp;
            a.visits = d_vis;
            // visited set: an LDS hash table (a query visits up to about
            // degree x ef points; the table holds 3/4 of its slots) or, when
            // that table would leave fewer than five waves per CU (S2 at
            // ef 200: one wave per SIMD, 19.0 ms against 10.7 ms), a bitmap
            // of N bits per wave in HBM with a few KiB of LDS per wave
            constexpr size_t kHashLdsMax = 32768;
            int H = p.visited_slots;
            bool bitmap_only = H == -1;
            if (H == 0) {
                const int64_t want = static_cast<int64_t>(degree) * ef * 4 / 3;
                H = 512;
                while (H < want && search_lds_bytes(a.CC, a.efr, a.Dp, 2 * H) <= 65536) H *= 2;
                bitmap_only = search_lds_bytes(a.CC, a.efr, a.Dp, H) > kHashLdsMax;
            }
            // queries (all, or those that outgrew the on-chip table) on the
            // bitmap path: up to kBitmapWaves waves, each clearing its bitmap
            // after every query
            auto run_bitmap = [&](const int32_t* d_list, int64_t n) {
                constexpr int64_t kBitmapWaves = 2048;   // S2, ef 200: 4096 and 8192 no faster
                const int64_t words = ceil_div(N, 32);
                const int64_t by_mem = std::max<int64_t>(1, (int64_t(4) << 30) / (words * 4));
                const int64_t slots = std::min<int64_t>({n, kBitmapWaves, by_mem});
                uint32_t* bmp = c.ws<uint32_t>(W_TMP, static_cast<size_t>(slots * words));
                GT_HIP(hipMemsetAsync(bmp, 0, static_cast<size_t>(slots * words) * 4, c.s));
                a.q_list = d_list;
                a.n_run = n;
                a.H = 0;
                a.bitmap = bmp;
                a.bm_words = words;
                GT_REQUIRE(search_lds_bytes(a.CC, a.efr, a.Dp, 0) <= 65536, "ef / dimension too large for one query's LDS");
                st.t_search += c.timed([&] { launch_graph_search(a, slots, c.s); });
            };
            std::vector<int32_t> hs(static_cast<size_t>(nq)), hx(static_cast<size_t>(nq)), hv(static_cast<size_t>(nq));
            if (bitmap_only) {
                run_bitmap(nullptr, nq);
                c.d2h(hs.data(), d_status, hs.size() * sizeof(int32_t));
                c.sync();
                for (int64_t q = 0; q < nq; ++q)
                    GT_REQUIRE(hs[static_cast<size_t>(q)] == 0,
                               "search: more candidates tie at the ef-th distance than fit (query " + std::to_string(q) + ")");
            } else {
                GT_REQUIRE(H >= 512 && (H & (H - 1)) == 0, "visited_slots must be -1, 0 or a power of two >= 512");
                GT_REQUIRE(search_lds_bytes(a.CC, a.efr, a.Dp, H) <= 65536, "ef / dimension too large for one query's LDS");
                a.H = H;
                st.t_search = c.timed([&] { launch_graph_search(a, nq, c.s); });
                c.d2h(hs.data(), d_status, hs.size() * sizeof(int32_t));
                c.sync();
                std::vector<int32_t> redo;
                for (int64_t q = 0; q < nq; ++q) {
                    GT_REQUIRE(hs[static_cast<size_t>(q)] != 2,
                               "search: more candidates tie at the ef-th distance than fit (query " + std::to_string(q) + ")");
                    if (hs[static_cast<size_t>(q)] == 1) redo.push_back(static_cast<int32_t>(q));
                }
                if (!redo.empty()) {
                    int32_t* d_redo = c.ws<int32_t>(W_QROWS, redo.size());
                    c.h2d(d_redo, redo.data(), redo.size() * sizeof(int32_t));
                    run_bitmap(d_redo, static_cast<int64_t>(redo.size()));
                    c.d2h(hs.data(), d_status, hs.size() * sizeof(int32_t));
                    c.sync();
                    for (int32_t q : redo)
                        GT_REQUIRE(hs[static_cast<size_t>(q)] == 0,
                                   "search: more candidates tie at the ef-th distance than fit (query " + std::to_string(q) + ")");
                    st.requeued = static_cast<int64_t>(redo.size());
                }
            }
            c.d2h(hx.data(), d_exp, hx.size() * sizeof(int32_t));
            c.d2h(hv.data(), d_vis, hv.size() * sizeof(int32_t));
            c.out(out_ids, oi, nr);
            c.out(out_d, od, nr);
            c.sync();
            for (int32_t x : hx) st.expansions += x;
            for (int32_t x : hv) st.visited += x;
        }
        st.t_total = tt.sec();
        if (stats) *stats = st;
    });
}

int gt_knn_exact(gt_ctx* ctx, const void* X, int64_t N, int32_t D, int dtype, int metric, const int64_t* queries,
                 int64_t nq, int32_t k, int32_t* ids, float* dists)
{
    return guarded(ctx, [&] {
        GT_REQUIRE(ids && dists && k >= 1 && k <= 128, "k must be in [1, 128]");
        GT_REQUIRE(metric == GT_METRIC_L2 || metric == GT_METRIC_IP, "unknown metric");
        GT_REQUIRE(queries || nq == N, "nq must equal N when queries is NULL");
        Ctx c(ctx);
        DevMatrix Xm = prepare(c, W_X, W_XRAW, W_NORMS, X, N, D, dtype, true, true);
        int32_t* d_q = nullptr;
        if (queries) {
            std::vector<int64_t> hq(static_cast<size_t>(nq));
            if (is_device_ptr(queries)) {
                c.d2h(hq.data(), queries, static_cast<size_t>(nq) * sizeof(int64_t));
                c.sync();
            } else {
                std::memcpy(hq.data(), queries, static_cast<size_t>(nq) * sizeof(int64_t));
            }
            std::vector<int32_t> q32(static_cast<size_t>(nq));
            for (int64_t i = 0; i < nq; ++i) {
                GT_REQUIRE(hq[static_cast<size_t>(i)] >= 0 && hq[static_cast<size_t>(i)] < N, "query id out of range");
                q32[static_cast<size_t>(i)] = static_cast<int32_t>(hq[static_cast<size_t>(i)]);
            }
            d_q = c.ws<int32_t>(W_QROWS, static_cast<size_t>(nq));
            c.h2d(d_q, q32.data(), q32.size() * sizeof(int32_t));
        }
        if (nq == 0) return;
        int32_t* oi = c.in<int32_t>(W_IDS, ids, static_cast<size_t>(nq) * k, false);
        float* od = c.in<float>(W_D, dists, static_cast<size_t>(nq) * k, false);
        KnnJob j;
        j.Q = &Xm;
        j.P = &Xm;
        j.q_rows = d_q;
        j.nq = nq;
        j.np = N;
        j.M = k;
        j.metric = metric;
        j.exclude_self = true;
        j.out_ids = oi;
        j.out_d = od;
        run_knn_flat(c, j);
        if (metric == GT_METRIC_IP) launch_negate(od, nq * k, c.s);
        c.out(ids, oi, static_cast<size_t>(nq) * k);
        c.out(dists, od, static_cast<size_t>(nq) * k);
        c.sync();
    });
}

int gt_assign_top2(gt_ctx* ctx, const void* X, int64_t N, int32_t D, int dtype, int metric, const void* C,
                   int64_t nC, uint32_t* top2, float* d2)
{
    return guarded(ctx, [&] {
        GT_REQUIRE(top2 && d2 && nC >= 1, "bad arguments");
        Ctx c(ctx);
        DevMatrix Xm = prepare(c, W_X, W_XRAW, W_NORMS, X, N, D, dtype);
        DevMatrix Cm = prepare(c, W_C, W_CRAW, W_CNORMS, C, nC, D, dtype);
        int32_t* oi = c.in<int32_t>(W_IDS, reinterpret_cast<int32_t*>(top2), static_cast<size_t>(N) * 2, false);
        float* od = c.in<float>(W_D, d2, static_cast<size_t>(N) * 2, false);
        KnnJob j;
        j.Q = &Xm;
        j.P = &Cm;
        j.nq = N;
        j.np = nC;
        j.M = 2;
        j.metric = metric;
        j.exclude_self = false;
        j.out_pos = true;
        j.out_ids = oi;
        j.out_d = od;
        run_knn_flat(c, j, 1);
        if (metric == GT_METRIC_IP) launch_negate(od, N * 2, c.s);
        c.out(reinterpret_cast<int32_t*>(top2), oi, static_cast<size_t>(N) * 2);
        c.out(d2, od, static_cast<size_t>(N) * 2);
        c.sync();
    });
}

int gt_knn_bucketed(gt_ctx* ctx, const void* X, int64_t N, int32_t D, int dtype, int metric, const int64_t* offsets,
                    const int32_t* members, int64_t nB, const int32_t* probe, int32_t P, int32_t M, int32_t* ids,
                    float* dists, int merge)
{
    return guarded(ctx, [&] {
        GT_REQUIRE(offsets && members && ids && dists && nB >= 1 && M >= 1 && M <= 128 && P >= 0, "bad arguments");
        GT_REQUIRE(P == 0 || probe, "probe table missing");
        Ctx c(ctx);
        Buckets b;
        b.offsets.resize(static_cast<size_t>(nB + 1));
        b.members.resize(static_cast<size_t>(N));
        b.probe.resize(static_cast<size_t>(nB) * P);
        b.P = P;
        auto fetch = [&](void* dst, const void* src, size_t bytes) {
            if (is_device_ptr(src)) { c.d2h(dst, src, bytes); c.sync(); }
            else std::memcpy(dst, src, bytes);
        };
        fetch(b.offsets.data(), offsets, b.offsets.size() * sizeof(int64_t));
        fetch(b.members.data(), members, b.members.size() * sizeof(int32_t));
        if (P > 0) fetch(b.probe.data(), probe, b.probe.size() * sizeof(int32_t));
        GT_REQUIRE(b.offsets[0] == 0 && b.offsets[static_cast<size_t>(nB)] == N, "offsets must span all N points");
        {
            std::vector<uint8_t> seen(static_cast<size_t>(N), 0);
            for (int64_t bb = 0; bb < nB; ++bb)
                GT_REQUIRE(b.offsets[static_cast<size_t>(bb + 1)] >= b.offsets[static_cast<size_t>(bb)], "offsets must be non-decreasing");
            for (int64_t i = 0; i < N; ++i) {
                const int32_t m = b.members[static_cast<size_t>(i)];
                GT_REQUIRE(m >= 0 && m < N && !seen[static_cast<size_t>(m)], "members must be a permutation of [0, N)");
                seen[static_cast<size_t>(m)] = 1;
            }
        }
        DevMatrix Xm = prepare(c, W_X, W_XRAW, W_NORMS, X, N, D, dtype, true, true);
        const size_t nm = static_cast<size_t>(N) * M;
        int32_t* cur_i = c.ws<int32_t>(W_IDS, nm);
        float* cur_d = c.ws<float>(W_D, nm);
        const float* seed = nullptr;
        int32_t* run_i = nullptr;
        float* run_d = nullptr;
        if (merge) {
            run_i = c.in<int32_t>(W_IDS2, ids, nm);
            run_d = c.in<float>(W_D2, dists, nm);
            if (metric == GT_METRIC_IP) {
                float* tmp = c.ws<float>(W_D3, nm);
                c.d2d(tmp, run_d, nm * sizeof(float));
                launch_negate(tmp, static_cast<int64_t>(nm), c.s);
                run_d = tmp;
            }
            seed = run_d;
        }
        bool merged = false;
        bucketed_round(c, Xm, b, M, metric, seed, cur_i, cur_d, nullptr, nullptr, nullptr, true, true, 0, -1, run_i,
                       &merged);
        int32_t* res_i = cur_i;
        float* res_d = cur_d;
        if (merged) {   // the collect launch merged the new lists into (run_i, run_d)
            res_i = run_i;
            res_d = run_d;
        } else if (merge) {
            int32_t* mi = c.ws<int32_t>(W_G1, nm);
            float* md = c.ws<float>(W_G2, nm);
            launch_merge_rounds(run_i, run_d, cur_i, cur_d, N, M, mi, md, c.s);
            res_i = mi;
            res_d = md;
        }
        if (metric == GT_METRIC_IP) launch_negate(res_d, static_cast<int64_t>(nm), c.s);
        c.out(ids, res_i, nm);
        c.out(dists, res_d, nm);
        c.sync();
    });
}

int gt_merge_rounds(gt_ctx* ctx, const int32_t* run_ids, const float* run_d, const int32_t* new_ids,
                    const float* new_d, int64_t N, int32_t M, int32_t* out_ids, float* out_d)
{
    return guarded(ctx, [&] {
        GT_REQUIRE(run_ids && run_d && new_ids && new_d && out_ids && out_d && N >= 0 && M >= 1 && M <= 128,
                   "bad arguments");
        Ctx c(ctx);
        const size_t nm = static_cast<size_t>(N) * M;
        const int32_t* ri = c.in<int32_t>(W_IDS, run_ids, nm);
        const float* rd = c.in<float>(W_D, run_d, nm);
        const int32_t* ni = c.in<int32_t>(W_IDS2, new_ids, nm);
        const float* nd = c.in<float>(W_D2, new_d, nm);
        int32_t* oi = c.ws<int32_t>(W_G1, nm);
        float* od = c.ws<float>(W_G2, nm);
        launch_merge_rounds(ri, rd, ni, nd, N, M, oi, od, c.s);
        c.out(out_ids, oi, nm);
        c.out(out_d, od, nm);
        c.sync();
    });
}

int gt_refine_2hop(gt_ctx* ctx, const void* X, int64_t N, int32_t D, int dtype, int metric, int32_t M, int32_t S,
                   int32_t passes, int32_t* ids, float* dists)
{
    return guarded(ctx, [&] {
        GT_REQUIRE(ids && dists && M >= 1 && M <= 128 && S >= 1 && S <= M && S * S <= 1024 && passes >= 0,
                   "bad arguments (need 1 <= S <= M, S*S <= 1024)");
        Ctx c(ctx);
        DevMatrix Xm = prepare(c, W_X, W_XRAW, W_NORMS, X, N, D, dtype);
        const size_t nm = static_cast<size_t>(N) * M;
        int32_t* ai = c.ws<int32_t>(W_IDS, nm);
        float* ad = c.ws<float>(W_D, nm);
        c.d2d(ai, c.in<int32_t>(W_IDS2, ids, nm), nm * sizeof(int32_t));
        c.d2d(ad, c.in<float>(W_D2, dists, nm), nm * sizeof(float));
        if (metric == GT_METRIC_IP) launch_negate(ad, static_cast<int64_t>(nm), c.s);
        int32_t* bi = c.ws<int32_t>(W_G1, nm);
        float* bd = c.ws<float>(W_G2, nm);
        for (int p = 0; p < passes; ++p) {
            launch_refine_2hop(Xm.data, Xm.norms, N, Xm.Dp, metric, nullptr, ai, ad, M, S, bi, bd, c.s);
            std::swap(ai, bi);
            std::swap(ad, bd);
        }
        if (metric == GT_METRIC_IP) launch_negate(ad, static_cast<int64_t>(nm), c.s);
        c.out(ids, ai, nm);
        c.out(dists, ad, nm);
        c.sync();
    });
}

int gt_sanitize(gt_ctx* ctx, const int32_t* knn, int64_t N, int32_t M, uint32_t* out)
{
    return guarded(ctx, [&] {
        GT_REQUIRE(knn && out && N >= 1 && M >= 1, "bad arguments");
        Ctx c(ctx);
        const size_t nm = static_cast<size_t>(N) * M;
        const int32_t* in = c.in<int32_t>(W_IN, knn, nm);
        uint32_t* o = c.ws<uint32_t>(W_OUT, nm);
        launch_sanitize(in, N, M, o, c.s);
        c.out(out, o, nm);
        c.sync();
    });
}

int gt_cagra_prune(gt_ctx* ctx, const uint32_t* knn, int64_t N, int32_t M, int32_t K, uint32_t* out)
{
    return guarded(ctx, [&] {
        GT_REQUIRE(knn && out && N >= 1 && M >= 1, "bad arguments");
        GT_REQUIRE(N < (int64_t(1) << 31), "N must be < 2^31");
        Ctx c(ctx);
        const size_t nm = static_cast<size_t>(N) * M;
        const uint32_t* in = c.in<uint32_t>(W_IN, knn, nm);
        uint32_t* o = c.ws<uint32_t>(W_OUT, static_cast<size_t>(N) * K);
        prune_device(c, reinterpret_cast<const int32_t*>(in), N, M, K, o);
        c.out(out, o, static_cast<size_t>(N) * K);
        c.sync();
    });
}

int gt_reverse_merge(gt_ctx* ctx, const uint32_t* fwd, int64_t N, int32_t K, uint32_t* out)
{
    return guarded(ctx, [&] {
        GT_REQUIRE(fwd && out && N >= 1 && K >= 1, "bad arguments");
        Ctx c(ctx);
        const size_t nk = static_cast<size_t>(N) * K;
        const uint32_t* in = c.in<uint32_t>(W_IN, fwd, nk);
        uint32_t* o = c.ws<uint32_t>(W_OUT, nk);
        reverse_merge_device(c, in, N, K, o);
        c.out(out, o, nk);
        c.sync();
    });
}

int gt_prune_occlusion(gt_ctx* ctx, const void* X, int64_t N, int32_t D, int dtype, const int32_t* nb, int32_t M,
                       int32_t max_degree, int32_t* out)
{
    return guarded(ctx, [&] {
        GT_REQUIRE(nb && out && M >= 1 && M <= 128, "bad arguments (1 <= M <= 128)");
        Ctx c(ctx);
        DevMatrix Xm = prepare(c, W_X, W_XRAW, W_NORMS, X, N, D, dtype);
        const size_t nm = static_cast<size_t>(N) * M;
        const int32_t* in = c.in<int32_t>(W_IN, nb, nm);
        int32_t* o = c.ws<int32_t>(W_OUT, nm);
        launch_occlusion_prune(Xm.data, N, Xm.Dp, in, M, max_degree, o, c.s);
        c.out(out, o, nm);
        c.sync();
    });
}

int gt_reverse_insert(gt_ctx* ctx, int32_t* ids, float* dists, int64_t N, int32_t M)
{
    return guarded(ctx, [&] {
        GT_REQUIRE(ids && dists && N >= 1 && M >= 1, "bad arguments");
        GT_REQUIRE(N < (int64_t(1) << 31), "N must be < 2^31");
        Ctx c(ctx);
        const size_t nm = static_cast<size_t>(N) * M;
        int32_t* di = c.in<int32_t>(W_IDS, ids, nm);
        float* dd = c.in<float>(W_D, dists, nm);
        reverse_insert_device(c, di, dd, N, M);
        c.out(ids, di, nm);
        c.out(dists, dd, nm);
        c.sync();
    });
}

int gt_optimize(gt_ctx* ctx, const uint32_t* knn, int64_t N, int32_t M, int32_t K, uint32_t* out)
{
    return guarded(ctx, [&] {
        GT_REQUIRE(knn && out && N >= 1 && M >= 1, "bad arguments");
        Ctx c(ctx);
        const size_t nm = static_cast<size_t>(N) * M, nk = static_cast<size_t>(N) * K;
        const uint32_t* in = c.in<uint32_t>(W_IN, knn, nm);
        uint32_t* f = c.ws<uint32_t>(W_G3, nk);
        prune_device(c, reinterpret_cast<const int32_t*>(in), N, M, K, f);
        uint32_t* o = c.ws<uint32_t>(W_OUT, nk);
        reverse_merge_device(c, f, N, K, o);
        c.out(out, o, nk);
        c.sync();
    });
}

int gt_optimize_noalloc(gt_ctx* ctx, const uint32_t* knn, int64_t N, int32_t M, int32_t K, uint32_t* out)
{
    return guarded(ctx, [&] {
        GT_REQUIRE(knn && out && N >= 1 && M >= 1 && M <= 128 && K >= 1 && K <= M && K <= 64,
                   "gt_optimize_noalloc: bad arguments (need 1 <= K <= min(M, 64), M <= 128)");
        GT_REQUIRE(N * K <= GT_NOALLOC_MAX_EDGES,
                   "gt_optimize_noalloc: N * K = " + std::to_string(N * K) + " edges exceeds the scratch maximum of " +
                       std::to_string(GT_NOALLOC_MAX_EDGES) + " (use gt_optimize)");
        GT_REQUIRE(on_device(knn, ctx->device) && on_device(out, ctx->device),
                   "gt_optimize_noalloc: knn and out must be device memory of the context's GPU");
        if (!ctx->scratch) throw Error(GT_EDEVICE, "gt_optimize_noalloc: no scratch array: " + ctx->scratch_err);
        const NoAllocLayout L = noalloc_layout(N, K);
        GT_REQUIRE(L.bytes <= GT_NOALLOC_SCRATCH_BYTES, "gt_optimize_noalloc: scratch layout too large");
        unsigned char* base = static_cast<unsigned char*>(ctx->scratch);
        auto at = [&](size_t off) { return static_cast<void*>(base + off); };
        uint32_t* fwd = static_cast<uint32_t*>(at(L.fwd));
        unsigned long long* bad = static_cast<unsigned long long*>(at(L.bad));
        int* err = static_cast<int*>(at(L.err));
        hipStream_t s = ctx->stream;
        // the array keeps the previous call's contents: reset the flags (a
        // kernel, not a memset node); everything else is written before it is read
        launch_init_flags(bad, err, s);
        launch_cagra_prune(reinterpret_cast<const int32_t*>(knn), N, M, K, fwd, bad, s, nullptr,
                           ctx->dbg.prune_flat_rows != 0);
        unsigned long long h_bad = 0;
        GT_HIP(hipMemcpyAsync(&h_bad, bad, sizeof(h_bad), hipMemcpyDeviceToHost, s));
        GT_HIP(hipStreamSynchronize(s));
        if (h_bad != ~0ull)
            throw Error(GT_EFEWCAND, "prune: row " + std::to_string(h_bad) +
                                         " has fewer than output_degree valid candidates");
        launch_rev_binned(fwd, N, K, static_cast<uint32_t*>(at(L.hist)), static_cast<uint32_t*>(at(L.offs)),
                          static_cast<uint32_t*>(at(L.sums)), static_cast<unsigned long long*>(at(L.part)),
                          static_cast<unsigned long long*>(at(L.grouped)), out, err, s);
        int h_err = 0;
        GT_HIP(hipMemcpyAsync(&h_err, err, sizeof(h_err), hipMemcpyDeviceToHost, s));
        GT_HIP(hipStreamSynchronize(s));
        if (h_err) throw Error(GT_EINVAL, "reverse merge: forward graph holds an id >= N");
    });
}

int gt_translate(gt_ctx* ctx, const uint32_t* g, const uint32_t* inv, int64_t N, int32_t K, uint32_t* out)
{
    return guarded(ctx, [&] {
        GT_REQUIRE(g && inv && out && N >= 1 && K >= 1, "bad arguments");
        Ctx c(ctx);
        const size_t nk = static_cast<size_t>(N) * K;
        const uint32_t* dg = c.in<uint32_t>(W_IN, g, nk);
        const uint32_t* dinv = c.in<uint32_t>(W_CUR, inv, static_cast<size_t>(N));
        uint32_t* o = c.ws<uint32_t>(W_OUT, nk);
        uint32_t* hits = c.ws<uint32_t>(W_DEG, static_cast<size_t>(N));
        int* err = c.ws<int>(W_TMP, 1);
        GT_HIP(hipMemsetAsync(hits, 0, static_cast<size_t>(N) * sizeof(uint32_t), c.s));
        GT_HIP(hipMemsetAsync(err, 0, sizeof(int), c.s));
        launch_translate(dg, dinv, N, K, o, hits, err, c.s);
        int h = 0;
        c.d2h(&h, err, sizeof(int));
        c.sync();
        if (h) throw Error(GT_EINVAL, "translate: ids out of range or inverse_perm is not a permutation");
        c.out(out, o, nk);
        c.sync();
    });
}

int gt_build_graph(gt_ctx* ctx, const void* X, int64_t N, int32_t D, int dtype, const gt_build_params* params,
                   int32_t* knn_ids, float* knn_dists, uint32_t* graph, gt_build_stats* stats)
{
    return gt_build_graph_ex(ctx, X, N, D, dtype, params, knn_ids, knn_dists, graph, stats, nullptr);
}

// Host-side DiskJoin processing order over a CSR bucket graph; the
// candidates live in a max-heap on (score, id) with one entry per bucket,
// updated in place as the window slides.
namespace {
class ScoreHeap {
public:
    explicit ScoreHeap(const std::vector<int64_t>& score) : sc_(score), at_(score.size(), -1) {}
    bool empty() const { return h_.empty(); }
    void touch(int32_t v)
    {
        if (at_[static_cast<size_t>(v)] < 0) {
            at_[static_cast<size_t>(v)] = static_cast<int32_t>(h_.size());
            h_.push_back(v);
        }
        up(at_[static_cast<size_t>(v)]);
        down(at_[static_cast<size_t>(v)]);
    }
    int32_t pop()
    {
        const int32_t top = h_[0];
        at_[static_cast<size_t>(top)] = -1;
        const int32_t last = h_.back();
        h_.pop_back();
        if (!h_.empty()) {
            h_[0] = last;
            at_[static_cast<size_t>(last)] = 0;
            down(0);
        }
        return top;
    }

private:
    bool above(int32_t a, int32_t b) const   // a before b: larger score, then larger id
    {
        const int64_t x = sc_[static_cast<size_t>(a)], y = sc_[static_cast<size_t>(b)];
        return x != y ? x > y : a > b;
    }
    void place(int32_t i, int32_t v)
    {
        h_[static_cast<size_t>(i)] = v;
        at_[static_cast<size_t>(v)] = i;
    }
    void up(int32_t i)
    {
        const int32_t v = h_[static_cast<size_t>(i)];
        while (i > 0) {
            const int32_t p = (i - 1) / 2;
            if (!above(v, h_[static_cast<size_t>(p)])) break;
            place(i, h_[static_cast<size_t>(p)]);
            i = p;
        }
        place(i, v);
    }
    void down(int32_t i)
    {
        const int32_t n = static_cast<int32_t>(h_.size());
        const int32_t v = h_[static_cast<size_t>(i)];
        for (;;) {
            int32_t c = 2 * i + 1;
            if (c >= n) break;
            if (c + 1 < n && above(h_[static_cast<size_t>(c + 1)], h_[static_cast<size_t>(c)])) ++c;
            if (!above(h_[static_cast<size_t>(c)], v)) break;
            place(i, h_[static_cast<size_t>(c)]);
            i = c;
        }
        place(i, v);
    }
    const std::vector<int64_t>& sc_;
    std::vector<int32_t> at_;
    std::vector<int32_t> h_;
};
}  // namespace

static std::vector<int32_t> diskjoin_order(const uint32_t* g, int64_t B, int32_t K, int32_t window)
{
    std::vector<int32_t> order;
    if (B <= 0) return order;
    order.reserve(static_cast<size_t>(B));
    window = std::max<int32_t>(1, window);
    // out-neighbours (row order, repeats kept) and their reverse lists
    std::vector<int64_t> ao(static_cast<size_t>(B + 1), 0), ro(static_cast<size_t>(B + 1), 0);
    std::vector<int32_t> adj;
    adj.reserve(static_cast<size_t>(B) * std::max(K, 0));
    for (int64_t v = 0; v < B; ++v) {
        for (int32_t k = 0; k < K; ++k) {
            const uint32_t u = g[static_cast<size_t>(v) * K + k];
            if (static_cast<int64_t>(u) != v && static_cast<int64_t>(u) < B) {
                adj.push_back(static_cast<int32_t>(u));
                ro[static_cast<size_t>(u) + 1]++;
            }
        }
        ao[static_cast<size_t>(v) + 1] = static_cast<int64_t>(adj.size());
    }
    for (int64_t u = 0; u < B; ++u) ro[static_cast<size_t>(u) + 1] += ro[static_cast<size_t>(u)];
    std::vector<int32_t> rev(adj.size());
    {
        std::vector<int64_t> cur(ro.begin(), ro.end() - 1);
        for (int64_t v = 0; v < B; ++v)
            for (int64_t e = ao[static_cast<size_t>(v)]; e < ao[static_cast<size_t>(v) + 1]; ++e)
                rev[static_cast<size_t>(cur[static_cast<size_t>(adj[static_cast<size_t>(e)])]++)] = static_cast<int32_t>(v);
    }
    int32_t start = 0;
    for (int64_t v = 1; v < B; ++v)
        if (ao[static_cast<size_t>(v) + 1] - ao[static_cast<size_t>(v)] >
            ao[static_cast<size_t>(start) + 1] - ao[static_cast<size_t>(start)])
            start = static_cast<int32_t>(v);
    std::vector<uint8_t> placed(static_cast<size_t>(B), 0);
    std::vector<int64_t> score(static_cast<size_t>(B), 0);   // summed neighbour overlap with the window
    ScoreHeap heap(score);
    auto slide = [&](int32_t p, int64_t delta) {
        for (int64_t e = ao[static_cast<size_t>(p)]; e < ao[static_cast<size_t>(p) + 1]; ++e) {
            const int32_t u = adj[static_cast<size_t>(e)];
            for (int64_t r = ro[static_cast<size_t>(u)]; r < ro[static_cast<size_t>(u) + 1]; ++r) {
                const int32_t v = rev[static_cast<size_t>(r)];
                if (placed[static_cast<size_t>(v)]) continue;
                score[static_cast<size_t>(v)] += delta;
                heap.touch(v);
            }
        }
    };
    int64_t lowest = 0;
    auto put = [&](int32_t v) {
        order.push_back(v);
        placed[static_cast<size_t>(v)] = 1;
        slide(v, +1);
    };
    put(start);
    for (int64_t i = 1; i < B; ++i) {
        if (i > window) slide(order[static_cast<size_t>(i - window - 1)], -1);
        int32_t pick;
        if (!heap.empty()) {
            pick = heap.pop();
        } else {
            while (placed[static_cast<size_t>(lowest)]) ++lowest;
            pick = static_cast<int32_t>(lowest);
        }
        put(pick);
    }
    return order;
}

int gt_bucket_order(gt_ctx* ctx, const uint32_t* graph, int64_t B, int32_t K, int32_t window, int32_t* order)
{
    return guarded_host(ctx, [&](gt_ctx* cx) {
        GT_REQUIRE(order && B >= 0 && B < (int64_t(1) << 31) && K >= 0 && (B == 0 || K == 0 || graph),
                   "bad arguments");
        std::vector<uint32_t> hg(static_cast<size_t>(B) * static_cast<size_t>(K));
        fetch_host(cx, hg.data(), graph, hg.size());
        const std::vector<int32_t> o = diskjoin_order(hg.data(), B, K, window);
        store_host(cx, order, o.data(), o.size());
    });
}

int gt_bucket_reorder(gt_ctx* ctx, const int32_t* assignment, int64_t N, int64_t n_buckets, const int32_t* order,
                      const int64_t* cids, int64_t n_cids, uint32_t* inverse_perm, uint32_t* bucket_offsets,
                      uint32_t* cids_new)
{
    return guarded_host(ctx, [&](gt_ctx* cx) {
        GT_REQUIRE(assignment && order && inverse_perm && bucket_offsets && N >= 1 && N < (int64_t(1) << 31) &&
                       n_buckets >= 1 && n_buckets < (int64_t(1) << 31) && n_cids >= 0 &&
                       (n_cids == 0 || (cids && cids_new)),
                   "bad arguments");
        std::vector<int32_t> ord(static_cast<size_t>(n_buckets)), asg(static_cast<size_t>(N));
        fetch_host(cx, ord.data(), order, ord.size());
        fetch_host(cx, asg.data(), assignment, asg.size());
        // processing position of every bucket; order must be a permutation
        std::vector<int32_t> pos(static_cast<size_t>(n_buckets), -1);
        for (int64_t q = 0; q < n_buckets; ++q) {
            const int32_t b = ord[static_cast<size_t>(q)];
            GT_REQUIRE(b >= 0 && b < n_buckets && pos[static_cast<size_t>(b)] < 0,
                       "order is not a permutation of the buckets");
            pos[static_cast<size_t>(b)] = static_cast<int32_t>(q);
        }
        std::vector<int32_t> key(static_cast<size_t>(N));
        std::atomic<int64_t> bad{-1};
        parallel_slices(N, host_threads(), [&](int, int64_t lo, int64_t hi) {
            for (int64_t i = lo; i < hi; ++i) {
                const int32_t b = asg[static_cast<size_t>(i)];
                if (b < 0 || b >= n_buckets) {
                    bad = i;
                    continue;
                }
                key[static_cast<size_t>(i)] = pos[static_cast<size_t>(b)];
            }
        });
        GT_REQUIRE(bad.load() < 0, "point " + std::to_string(bad.load()) + " has no bucket in [0, n_buckets)");
        // new ids: buckets in processing order, each bucket's points in old-id order
        std::vector<int32_t> inv(static_cast<size_t>(N));
        std::vector<int64_t> off;
        counting_sort(nullptr, N, key.data(), n_buckets, inv.data(), off);
        const std::vector<uint32_t> off32(off.begin(), off.end());
        store_host(cx, inverse_perm, reinterpret_cast<const uint32_t*>(inv.data()), inv.size());
        store_host(cx, bucket_offsets, off32.data(), off32.size());
        if (n_cids > 0) {
            std::vector<uint32_t> perm(static_cast<size_t>(N));
            parallel_slices(N, host_threads(), [&](int, int64_t lo, int64_t hi) {
                for (int64_t n = lo; n < hi; ++n)
                    perm[static_cast<size_t>(inv[static_cast<size_t>(n)])] = static_cast<uint32_t>(n);
            });
            std::vector<int64_t> hc(static_cast<size_t>(n_cids));
            fetch_host(cx, hc.data(), cids, hc.size());
            std::vector<uint32_t> out(static_cast<size_t>(n_cids));
            for (int64_t k = 0; k < n_cids; ++k) {
                const int64_t o = hc[static_cast<size_t>(k)];
                out[static_cast<size_t>(k)] = (o >= 0 && o < N) ? perm[static_cast<size_t>(o)] : 0xFFFFFFFFu;
            }
            store_host(cx, cids_new, out.data(), out.size());
        }
    });
}

// inverse_perm on the device, checked to be a permutation; perm (old -> new) on request
static const uint32_t* checked_perm(Ctx& c, const uint32_t* inverse_perm, int64_t N, uint32_t** perm_out)
{
    const uint32_t* dinv = c.in<uint32_t>(W_CUR, inverse_perm, static_cast<size_t>(N));
    uint32_t* perm = c.ws<uint32_t>(W_OFF, static_cast<size_t>(N));
    uint32_t* hits = c.ws<uint32_t>(W_DEG, static_cast<size_t>(N));
    int* err = c.ws<int>(W_FLAG, 1);
    GT_HIP(hipMemsetAsync(hits, 0, static_cast<size_t>(N) * sizeof(uint32_t), c.s));
    GT_HIP(hipMemsetAsync(err, 0, sizeof(int), c.s));
    launch_invert_perm(dinv, N, perm, hits, err, c.s);
    int h = 0;
    c.d2h(&h, err, sizeof(int));
    c.sync();
    if (h) throw Error(GT_EINVAL, "inverse_perm is not a permutation of [0, N)");
    if (perm_out) *perm_out = perm;
    return dinv;
}

int gt_permute_rows(gt_ctx* ctx, const void* X, int64_t N, int32_t D, int dtype, const uint32_t* inverse_perm,
                    void* out)
{
    return guarded(ctx, [&] {
        GT_REQUIRE(X && inverse_perm && out && N >= 1 && N < (int64_t(1) << 32) && D >= 1, "bad arguments");
        GT_REQUIRE(dtype == GT_DTYPE_F32 || dtype == GT_DTYPE_U8 || dtype == GT_DTYPE_I8, "unknown dtype");
        Ctx c(ctx);
        const int64_t rb = static_cast<int64_t>(D) * static_cast<int64_t>(dtype_size(dtype));
        const size_t bytes = static_cast<size_t>(N) * static_cast<size_t>(rb);
        const uint32_t* dinv = checked_perm(c, inverse_perm, N, nullptr);
        const uint8_t* dx = c.in<uint8_t>(W_XRAW, static_cast<const uint8_t*>(X), bytes);
        uint8_t* o = c.in<uint8_t>(W_TMP, static_cast<uint8_t*>(out), bytes, false);
        launch_permute_rows(dx, dinv, N, rb, o, c.s);
        c.out(static_cast<uint8_t*>(out), o, bytes);
        c.sync();
    });
}

int gt_remap_table(gt_ctx* ctx, const int32_t* ids, int64_t N, int32_t M, const uint32_t* inverse_perm, int32_t* out)
{
    return guarded(ctx, [&] {
        GT_REQUIRE(ids && inverse_perm && out && N >= 1 && N < (int64_t(1) << 31) && M >= 1, "bad arguments");
        Ctx c(ctx);
        const size_t nm = static_cast<size_t>(N) * M;
        uint32_t* perm = nullptr;
        const uint32_t* dinv = checked_perm(c, inverse_perm, N, &perm);
        const int32_t* di = c.in<int32_t>(W_IN, ids, nm);
        int32_t* o = c.in<int32_t>(W_OUT, out, nm, false);
        launch_remap_table(di, dinv, perm, N, M, o, c.s);
        c.out(out, o, nm);
        c.sync();
    });
}

int gt_build_graph_ex(gt_ctx* ctx, const void* X, int64_t N, int32_t D, int dtype, const gt_build_params* params,
                      int32_t* knn_ids, float* knn_dists, uint32_t* graph, gt_build_stats* stats,
                      const gt_build_extras* extras)
{
    return guarded(ctx, [&] {
        GT_REQUIRE(params && (graph || knn_ids || knn_dists), "bad arguments");
        gt_build_params p = *params;
        GT_REQUIRE(p.metric == GT_METRIC_L2 || p.metric == GT_METRIC_IP, "unknown metric");
        GT_REQUIRE(p.M >= 1 && p.M <= 128 && p.rounds >= 1, "bad degrees");
        GT_REQUIRE(!graph || (p.K >= 1 && p.K <= std::min(p.M, 64)), "bad output degree");
        GT_REQUIRE(N > p.M, "need N > M");
        Timer total;
        gt_build_stats st{};
        Ctx c(ctx);
        int64_t C = p.n_buckets > 0 ? p.n_buckets : std::max<int64_t>(1, N / 4000);
        C = std::min<int64_t>(C, N);
        // every round's random draws, one worker thread per round, while the
        // dataset is prepared
        std::vector<std::future<RoundSamples>> draws_jobs;
        for (int r = 0; r < p.rounds; ++r)
            draws_jobs.push_back(std::async(std::launch::async, [N, C, p, r] {
                return draw_round(N, C, p, p.seed + static_cast<uint64_t>(r));
            }));
        Timer tp;
        DevMatrix Xm = prepare(c, W_X, W_XRAW, W_NORMS, X, N, D, dtype, true, p.int_exact != 0);
        c.sync();
        st.t_prepare = tp.sec();
        std::vector<RoundSamples> draws;
        for (auto& j : draws_jobs) draws.push_back(j.get());
        int nprobe = p.nprobe;
        if (nprobe < 0) nprobe = static_cast<int>(std::ceil(20000.0 / (static_cast<double>(N) / C)));
        nprobe = static_cast<int>(std::min<int64_t>(nprobe, C - 1));

        const size_t nm = static_cast<size_t>(N) * p.M;
        // out of core when a device budget is set and the resident tables
        // (three N x M tables of ids and distances, the collect candidates,
        // the sanitized table and two graphs) exceed it
        const size_t budget = static_cast<size_t>(std::max(p.device_budget_mb, 0)) << 20;
        const size_t resident = nm * 4 * 7 + static_cast<size_t>(N) * kCollectCap * 8 +
                                (graph ? static_cast<size_t>(N) * p.K * 8 : 0);
        const bool ooc = budget > 0 && resident > budget;
        GT_REQUIRE(!ooc || (p.refine_passes == 0 && !p.reverse_edges),
                   "the out-of-core build (device budget below the tables) supports neither refinement nor "
                   "per-round reverse-edge insertion");
        std::vector<int32_t> h_run_i(ooc ? nm : 0);
        std::vector<float> h_run_d(ooc ? nm : 0);
        OocReport rep;
        int32_t* run_i = ooc ? nullptr : c.ws<int32_t>(W_G1, nm);
        float* run_d = ooc ? nullptr : c.ws<float>(W_G2, nm);
        int32_t* cur_i = ooc ? nullptr : c.ws<int32_t>(W_IDS, nm);
        float* cur_d = ooc ? nullptr : c.ws<float>(W_D, nm);
        int32_t* tmp_i = ooc ? nullptr : c.ws<int32_t>(W_IDS2, nm);
        float* tmp_d = ooc ? nullptr : c.ws<float>(W_D2, nm);
        ctx->knn_launches = 0;
        ctx->knn_pairs_done = 0.0;
        // a pass seeded with the running table's M-th distances, its lists
        // merged into the table: in place by the collect launch (only rows
        // with keys touched), else into (cur_i, cur_d) and then merged
        auto seeded = [&](const Buckets& b, bool own, bool probes) {
            bool merged = false;
            st.t_knn += bucketed_round(c, Xm, b, p.M, p.metric, run_d, cur_i, cur_d, &st.max_pool, &st.max_bucket,
                                       &st.knn_pairs, own, probes, 0, -1, run_i, &merged);
            if (merged) return;
            st.t_merge += c.timed([&] { launch_merge_rounds(run_i, run_d, cur_i, cur_d, N, p.M, tmp_i, tmp_d, c.s); });
            std::swap(run_i, tmp_i);
            std::swap(run_d, tmp_d);
        };
        // Round r's bucketing = bucket_device (device work + downloads, on
        // this thread) then bucket_host (two-choice + CSR, on a worker
        // thread).  The host half of round r runs while the device computes
        // round r+1's centroids and top-2 lists, and the host half of round
        // r+1 while the device runs round r's kNN; every device stage stays
        // on the context's stream in one order.
        Buckets bk[2];
        BucketPlan plans[2];
        for (int i = 0; i < 2; ++i) {
            bk[i].members.swap(ctx->h_members[i]);   // reuse host memory across builds
            bk[i].uploaded = ctx->members_up[i];
        }
        std::vector<int32_t> cknn;
        const bool want_cknn = extras && extras->centroid_knn && extras->centroid_knn_k > 0;
        auto device_part = [&](int r) {
            Timer tb;
            bucket_device(c, Xm, C, nprobe, p.metric, p.kmeans_iters, std::move(draws[static_cast<size_t>(r)]),
                          ctx->pinned[r & 1], plans[r & 1], r & 1, r == 0 && want_cknn ? &cknn : nullptr,
                          r == 0 && want_cknn ? extras->centroid_knn_k : 0);
            st.t_bucketing += tb.sec();
        };
        // the members' order (bucket, other top-2 centroid, id) is computed on
        // the device from the round's top-2 lists and the host's two-choice
        // buckets (the host half then only runs the sequential rule), except
        // out of core, where the host keeps the members, and where the debug
        // options ask for the host
        const bool dev_csr = !ooc && C >= 2 && C <= 16384 && c.c->dbg.bucket_host_csr == 0;
        auto bucket_of_host = [&](int r) { return ctx->pin_bucket[r & 1].as<int32_t>(static_cast<size_t>(N)); };
        std::future<void> host_job;   // declared after everything it references
        auto start_host = [&](int r) {
            // the previous upload of these buckets (two rounds ago) has been
            // read before the host half rewrites them
            GT_HIP(hipEventSynchronize(bk[r & 1].uploaded));
            int32_t* bo = bucket_of_host(r);
            host_job = std::async(std::launch::async, [&, r, bo] {
                bucket_host(plans[r & 1], p.balance, bk[r & 1], bo, !dev_csr, ctx->h_key2, ctx->h_by_key, ctx->h_bkt);
            });
        };
        // round r's members into W_MEMBERS and its offsets to the host
        auto device_csr = [&](int r) {
            Timer tc;
            Buckets& b = bk[r & 1];
            int32_t* d_bucket = c.ws<int32_t>(W_BUCKETD, static_cast<size_t>(N));
            c.h2d(d_bucket, bucket_of_host(r), static_cast<size_t>(N) * sizeof(int32_t));
            if (b.uploaded) GT_HIP(hipEventRecord(b.uploaded, c.s));
            const int64_t nh = C * csr_blocks(N);
            int32_t* d_mem = c.ws<int32_t>(W_MEMBERS, static_cast<size_t>(N));
            int64_t* d_off = c.ws<int64_t>(W_BOFF, static_cast<size_t>(C + 1));
            launch_bucket_csr(plans[r & 1].d_top2, d_bucket, N, static_cast<int>(C), c.ws<int32_t>(W_KEY2, static_cast<size_t>(N)),
                              c.ws<int32_t>(W_BYKEY, static_cast<size_t>(N)), c.ws<int32_t>(W_BKTD, static_cast<size_t>(N)),
                              c.ws<uint32_t>(W_LHIST, static_cast<size_t>(nh)),
                              c.ws<uint32_t>(W_LOFFS, static_cast<size_t>(nh + 1)),
                              c.ws<uint32_t>(W_LSUMS, static_cast<size_t>(nh / 1024 + 2)), d_mem, d_off, c.s);
            b.offsets.resize(static_cast<size_t>(C + 1));
            c.d2h(b.offsets.data(), d_off, static_cast<size_t>(C + 1) * sizeof(int64_t));
            c.sync();
            GT_REQUIRE(b.offsets[0] == 0 && b.offsets[static_cast<size_t>(C)] == N, "device bucket CSR");
            c.c->members_gen = b.gen;   // W_MEMBERS holds these buckets' members
            st.t_bucketing += tc.sec();
        };
        device_part(0);
        start_host(0);
        for (int r = 0; r < p.rounds; ++r) {
            if (r + 1 < p.rounds) device_part(r + 1);
            {
                Timer tw;
                host_job.get();   // rethrows the host half's errors
                st.t_bucketing += tw.sec();
            }
            if (dev_csr && plans[r & 1].d_top2) device_csr(r);
            GT_REQUIRE(!dev_csr || plans[r & 1].d_top2, "device bucket CSR without device top-2 lists");
            if (r == 0 && extras) {
                if (extras->round1_bucket) {
                    const int32_t* bo = bucket_of_host(r);
                    if (is_device_ptr(extras->round1_bucket)) c.h2d(extras->round1_bucket, bo, static_cast<size_t>(N) * sizeof(int32_t));
                    else std::memcpy(extras->round1_bucket, bo, static_cast<size_t>(N) * sizeof(int32_t));
                }
                if (want_cknn) {
                    if (is_device_ptr(extras->centroid_knn)) c.h2d(extras->centroid_knn, cknn.data(), cknn.size() * sizeof(int32_t));
                    else std::memcpy(extras->centroid_knn, cknn.data(), cknn.size() * sizeof(int32_t));
                }
                c.sync();
            }
            if (r + 1 == p.rounds && extras && (extras->last_bucket || extras->last_centroids)) {
                if (extras->last_bucket) {
                    const int32_t* bo = bucket_of_host(r);
                    if (is_device_ptr(extras->last_bucket)) c.h2d(extras->last_bucket, bo, static_cast<size_t>(N) * sizeof(int32_t));
                    else std::memcpy(extras->last_bucket, bo, static_cast<size_t>(N) * sizeof(int32_t));
                }
                if (extras->last_centroids) {
                    const std::vector<int32_t>& cid = plans[r & 1].cid;
                    std::vector<int64_t> w(cid.begin(), cid.end());
                    if (is_device_ptr(extras->last_centroids)) c.h2d(extras->last_centroids, w.data(), w.size() * sizeof(int64_t));
                    else std::memcpy(extras->last_centroids, w.data(), w.size() * sizeof(int64_t));
                }
                c.sync();
            }
            if (r + 1 < p.rounds) start_host(r + 1);
            const Buckets& b = bk[r & 1];
            if (ooc) {
                ooc_round(c, Xm, b, p.M, p.metric, r, h_run_i.data(), h_run_d.data(), budget, st, &rep);
                continue;
            }
            if (p.reverse_edges) {
                // the Python pipeline's round: full table, reverse edges, then the merge
                int32_t* oi = r == 0 ? run_i : cur_i;
                float* od = r == 0 ? run_d : cur_d;
                st.t_knn += bucketed_round(c, Xm, b, p.M, p.metric, nullptr, oi, od, &st.max_pool, &st.max_bucket,
                                           &st.knn_pairs);
                st.t_merge += c.timed([&] { reverse_insert_device(c, oi, od, N, p.M); });
                if (r > 0) {
                    st.t_merge += c.timed([&] { launch_merge_rounds(run_i, run_d, cur_i, cur_d, N, p.M, tmp_i, tmp_d, c.s); });
                    std::swap(run_i, tmp_i);
                    std::swap(run_d, tmp_d);
                }
            } else if (r == 0 && b.P > 0) {
                // the own buckets unseeded, then the probe buckets seeded with
                // that table's M-th distance, merged (disjoint candidate sets:
                // the same table as one pass over the whole pools)
                st.t_knn += bucketed_round(c, Xm, b, p.M, p.metric, nullptr, run_i, run_d, &st.max_pool,
                                           &st.max_bucket, &st.knn_pairs, true, false);
                seeded(b, false, true);
            } else if (r == 0) {
                st.t_knn += bucketed_round(c, Xm, b, p.M, p.metric, nullptr, run_i, run_d, &st.max_pool,
                                           &st.max_bucket, &st.knn_pairs);
            } else {
                seeded(b, true, true);
            }
        }
        for (int i = 0; i < 2; ++i) bk[i].members.swap(ctx->h_members[i]);
        if (ooc) {
            st.knn_flops = 2.0 * D * st.knn_pairs;
            st.knn_launches = ctx->knn_launches;
            st.knn_pairs_computed = ctx->knn_pairs_done;
            st.knn_int8 = use_i8(Xm, Xm, p.metric) ? 1 : 0;
            if (graph) {
                Timer t1;
                std::vector<uint32_t> san(nm), fwd(static_cast<size_t>(N) * p.K);
                sanitize_host(h_run_i.data(), N, p.M, san.data());
                prune_chunked(c, san.data(), N, p.M, p.K, budget, fwd.data(), &rep);
                st.t_prune = t1.sec();
                Timer t2;
                std::vector<uint32_t> fin(static_cast<size_t>(N) * p.K);
                reverse_merge_chunked(c, fwd.data(), N, p.K, budget, fin.data(), &rep);
                st.t_revmerge = t2.sec();
                if (is_device_ptr(graph)) c.h2d(graph, fin.data(), fin.size() * sizeof(uint32_t));
                else std::memcpy(graph, fin.data(), fin.size() * sizeof(uint32_t));
            }
            Timer td;
            if (p.metric == GT_METRIC_IP)
                for (float& v : h_run_d) v = -v;
            if (knn_ids) {
                if (is_device_ptr(knn_ids)) c.h2d(knn_ids, h_run_i.data(), nm * sizeof(int32_t));
                else std::memcpy(knn_ids, h_run_i.data(), nm * sizeof(int32_t));
            }
            if (knn_dists) {
                if (is_device_ptr(knn_dists)) c.h2d(knn_dists, h_run_d.data(), nm * sizeof(float));
                else std::memcpy(knn_dists, h_run_d.data(), nm * sizeof(float));
            }
            c.sync();
            st.t_download = td.sec();
            st.ooc_chunks = rep.chunks;
            st.t_total = total.sec();
            if (stats) *stats = st;
            return;
        }
        // refinement and the prune take the points in the last bucketing's
        // member order (W_MEMBERS holds it after a bucketed round): the rows
        // they gather (2-hop candidates, neighbour lists) sit mostly in the
        // point's own bucket, so they stay in L2
        const int32_t* order = c.c->members_gen != 0 ? c.ws<int32_t>(W_MEMBERS, static_cast<size_t>(N)) : nullptr;
        if (p.refine_passes > 0) {
            GT_REQUIRE(p.refine_sample >= 1 && p.refine_sample <= p.M && p.refine_sample * p.refine_sample <= 1024,
                       "bad refine sample");
            for (int pass = 0; pass < p.refine_passes; ++pass) {
                st.t_refine += c.timed([&] {
                    launch_refine_2hop(Xm.data, Xm.norms, N, Xm.Dp, p.metric, order, run_i, run_d, p.M,
                                       p.refine_sample, tmp_i, tmp_d, c.s);
                });
                std::swap(run_i, tmp_i);
                std::swap(run_d, tmp_d);
            }
        }
        st.knn_flops = 2.0 * D * st.knn_pairs;
        st.knn_launches = ctx->knn_launches;
        st.knn_pairs_computed = ctx->knn_pairs_done;
        st.knn_int8 = use_i8(Xm, Xm, p.metric) ? 1 : 0;
        // sanitize + prune + reverse merge
        uint32_t* fin = nullptr;
        if (graph) {
            uint32_t* san = c.ws<uint32_t>(W_OUT, nm);
            uint32_t* fwd = c.ws<uint32_t>(W_G3, static_cast<size_t>(N) * p.K);
            fin = c.ws<uint32_t>(W_IN, static_cast<size_t>(N) * p.K);
            const StageFlags fl = stage_flags(c);
            st.t_prune = c.timed([&] {
                launch_sanitize(run_i, N, p.M, san, c.s);
                prune_enqueue(c, fl, reinterpret_cast<const int32_t*>(san), N, p.M, p.K, fwd, order);
            });
            prune_check(c, fl);
            st.t_revmerge = c.timed([&] { reverse_merge_enqueue(c, fl, fwd, N, p.K, fin); });
            st.t_revmerge += reverse_merge_check(c, fl, fwd, N, p.K, fin);
        }
        Timer td;
        if (knn_ids) c.out(knn_ids, run_i, nm);
        if (knn_dists) {
            if (p.metric == GT_METRIC_IP) launch_negate(run_d, static_cast<int64_t>(nm), c.s);
            c.out(knn_dists, run_d, nm);
        }
        if (graph) c.out(graph, fin, static_cast<size_t>(N) * p.K);
        c.sync();
        st.t_download = td.sec();
        st.t_total = total.sec();
        if (stats) *stats = st;
    });
}

}  // extern "C"
