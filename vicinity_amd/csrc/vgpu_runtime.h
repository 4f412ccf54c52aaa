// Host runtime: device buffers, HIP error mapping and the IVF-PQ / flat index
// objects behind the C ABI.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <memory>
#include <mutex>
#include <shared_mutex>
#include <stdexcept>
#include <string>
#include <unordered_map>
#include <vector>

#include "../../include/vicinity_gpu.h"
#include "vgpu_launch.h"

namespace vgpu {

// Error carrying a vicinity status code; caught at the C ABI boundary.
struct Error : std::runtime_error {
    int code;
    Error(int c, const std::string& m) : std::runtime_error(m), code(c) {}
};

void hip_check(hipError_t e, const char* what);
#define VGPU_HIP(expr) ::vgpu::hip_check((expr), #expr)

// Device-allocation failure injection, a test hook: once armed with
// (after, count), the next `after` DevBuf allocations go through and the
// `count` after them fail as out-of-memory without calling hipMalloc.
void arm_alloc_failures(long long after, long long count);
bool alloc_should_fail();

template <typename T>
struct DevBuf {
    T* p = nullptr;
    size_t n = 0;
    DevBuf() = default;
    DevBuf(const DevBuf&) = delete;
    DevBuf& operator=(const DevBuf&) = delete;
    ~DevBuf() { release(); }
    void release() {
        if (p) (void)hipFree(p);
        p = nullptr;
        n = 0;
    }
    size_t bytes() const { return p ? n * sizeof(T) : 0; }
    // Grow-only allocation (contents are not preserved on growth).
    void reserve(size_t count) {
        if (count <= n && p) return;
        release();
        size_t bytes = (count ? count : 1) * sizeof(T);
        if (alloc_should_fail())
            throw Error(VGPU_ERR_OUT_OF_MEMORY,
                        "device allocation of " + std::to_string(bytes) + " bytes failed (injected)");
        hipError_t e = hipMalloc((void**)&p, bytes);
        if (e != hipSuccess) {
            p = nullptr;
            (void)hipGetLastError();
            throw Error(VGPU_ERR_OUT_OF_MEMORY,
                        "device allocation of " + std::to_string(bytes) + " bytes failed");
        }
        n = count;
    }
    void upload(const T* h, size_t count, hipStream_t s) {
        reserve(count);
        if (count) VGPU_HIP(hipMemcpyAsync(p, h, count * sizeof(T), hipMemcpyHostToDevice, s));
    }
};

// Sizes of one search call's device workspace: per query chunk, the
// normalised queries, coarse candidates or score rows, probe lists, scan
// results and statistics rows, plus the per-call scalars.
struct SearchPlan {
    size_t P = 0;      // probes per query (after min(nprobe, L))
    size_t kout = 0;   // results the scan keeps per query (k, or the rerank pool)
    size_t k = 0;      // results returned per query
    size_t pool = 0;   // rerank pool (0: no rerank)
    size_t chunk = 0;  // queries per launch sequence
    bool fused = false, opq = false;
    bool t2 = false;   // FAST scan tables from the MFMA pre-pass (chunk * M * 256 floats)
    // nprobe above 1024 or kout above 2048: probes chosen from exact scores of
    // every list, scans in EXACT (or FastScan) mode with per-slot list reads
    bool wide = false;
};

// Device pointers of one call's workspace, carved from one arena
// (ws_layout): a pooled SearchWs arena, or the static scratch of the
// allocation-free entry point.
struct WsPtrs {
    float *qn = nullptr, *qnorm = nullptr, *dots = nullptr, *dist = nullptr, *dist2 = nullptr,
          *rres = nullptr, *t2 = nullptr;
    uint32_t *cflag_list = nullptr, *probe = nullptr,
             *vidx = nullptr, *vidx2 = nullptr, *qstat = nullptr, *flag_list = nullptr;
    uint32_t* qbad = nullptr;  // per chunk query: 1 when the query holds a NaN or an infinity
    float* fdots = nullptr;  // coarse fallback: dot-product rows of the first flagged queries
    unsigned long long* scal = nullptr;  // per-call scalars (counters, flag-list lengths)
};

// Per-call device scalars: counter i at word i * COUNTER_STRIDE, then the
// overflow count and the two flag-list lengths, each on a cache line of its own,
// the coarse fallback's slice counters and the count of non-finite queries.
constexpr size_t kOverflowWord = (NUM_SCAN_COUNTERS + 1) * COUNTER_STRIDE;
constexpr size_t kFlagWord = kOverflowWord + 8;
constexpr size_t kCFlagWord = kFlagWord + 8;
constexpr size_t kFDoneWord = kCFlagWord + 8;  // COARSE_FLAG_PAR uint32 slice counters
constexpr size_t kBadWord = kFDoneWord + (COARSE_FLAG_PAR / 2 + 7) / 8 * 8;  // non-finite queries
constexpr size_t kScalWords = kBadWord + 8;

// Workspace of one search call.  A handle keeps a pool of these: each call
// borrows one for its whole duration, so concurrent searches on one handle
// use separate buffers and, unless the caller passes a stream, separate
// streams.  The arena grows to the largest plan seen and is reused.
struct SearchWs {
    hipStream_t stream = nullptr;
    hipEvent_t ev[9] = {};
    std::vector<hipEvent_t> sev;  // scan-only timing: four per chunk (scan kernel, table pre-pass)
    DevBuf<uint8_t> arena;
    DevBuf<float> q, odist;       // host-buffer entry points: staged queries and distances
    DevBuf<int64_t> ids;          // host-buffer entry points: staged ids
    DevBuf<uint32_t> slots;       // filtered search: per-query list slots
    DevBuf<uint8_t> want;         // filtered search: per-query category
    DevBuf<float> fqn, fdist, frres;  // filtered search: queries, distances, rotated residuals
    DevBuf<uint32_t> fvidx;           // filtered search: insertion indices
    DevBuf<uint32_t> gprobe;          // given probe lists (file-backed search)
    unsigned long long* h_scal = nullptr;  // pinned host copy of the per-call scalars
    SearchWs();
    ~SearchWs();
    SearchWs(const SearchWs&) = delete;
    SearchWs& operator=(const SearchWs&) = delete;
};

// A built IVF-PQ index.  Mirrors the state of IVFPQIndex
// (src/ivf_pq/search.rs:212-239): the raw normalised vectors and doc ids on
// the host, the search arrays resident in HBM.
//
// Locking: searches, probes and reads take `mu` shared (the reference's
// search takes &self, so concurrent searches are legal); add, build, load
// and setters take it exclusively (the reference's &mut self methods).
struct IvfpqIndex {
    size_t d = 0;
    vgpu_ivfpq_params params{};
    int device = 0;  // the HIP device current at construction
    int mode = VGPU_MODE_FAST;
    bool built = false;
    bool has_vectors = true;
    int profiling = 0;  // 0 off, 1 every phase, 2 the scan kernel only

    std::vector<float> vectors;     // [n*d] normalised (search.rs:503-508)
    std::vector<uint32_t> doc_ids;  // [n]

    size_t L = 0, K = 0, M = 0, ds = 0;
    std::vector<float> centroids;   // [L*d]
    std::vector<float> codebooks;   // [M*K*ds]
    std::vector<uint64_t> offsets;  // [L+1]
    std::vector<uint32_t> list_ids; // [n]
    std::vector<uint8_t> codes;     // [n*M] insertion order
    std::vector<float> rotation;    // [d*d] OPQ rotation R, row-major (opq.rs:37-38);
                                    // empty: Quantizer::Product

    hipStream_t stream = nullptr;   // build, upload and the allocation-free search
    DevBuf<float> d_centroids, d_codebooks, d_bias, d_vectors, d_rotation;
    DevBuf<uint4> d_cb16;           // bf16 hi/lo centroid copy of the search index
    DevBuf<uint32_t> d_offsets, d_list_ids, d_doc_ids, d_pack_off;
    DevBuf<uint8_t> d_codes, d_packed, d_tblocks;
    DevBuf<uint32_t> d_tblk_off;
    DevIndex dix;

    // build workspace (k-means assignment), used under the exclusive lock
    DevBuf<uint4> b_cb16;
    DevBuf<float> b_dots;
    DevBuf<uint32_t> b_cflag_list, b_cflag_count;
    DevBuf<unsigned int> b_overflow;

    std::shared_mutex mu;
    std::mutex pool_mu;                              // the free workspaces
    std::vector<std::unique_ptr<SearchWs>> ws_pool;
    std::mutex stats_mu;                             // stats of the last finished search
    vgpu_search_stats stats{};

    // search_with_filter state (search.rs:236-238): the category each document
    // carries in the filter field, per-list bitmasks taken when the lists are
    // built (search.rs:626-648), and device copies refreshed on demand (under
    // cat_mu, by the first filtered search after a change).
    bool filtering = false;
    std::unordered_map<uint32_t, int> doc_cat;  // doc id -> 0..63, or -1 (metadata without the field)
    std::vector<uint64_t> list_mask;            // [L]
    std::vector<uint32_t> list_cat_n;           // [L*64] entries per (list, category), current metadata
    bool cat_dirty = true;
    std::mutex cat_mu;
    DevBuf<uint8_t> d_ecat;  // category of each list-major entry (0xff: none)

    IvfpqIndex(size_t dim, const vgpu_ivfpq_params& p);
    ~IvfpqIndex();

    size_t n() const { return doc_ids.size(); }
    void add(const uint32_t* ids, const float* x, size_t count);
    void build(size_t sample, size_t max_iter);
    void load(const float* cent, size_t Lc, const float* cb, size_t Kc, const uint64_t* off,
              const uint32_t* lids, const uint8_t* cds, const uint32_t* dids, const float* vecs,
              size_t nv);
    void upload_index();
    // The rotation of an OPQ index built elsewhere (before load); null clears it.
    void set_rotation(const float* R);
    // The probe count, plan and shape checks of a search of nq queries.
    SearchPlan plan_search(size_t nq, size_t k, size_t nprobe, size_t pool) const;
    // Bytes of a plan's workspace arena; with a base, also the pointers into it.
    size_t ws_layout(const SearchPlan& pl, uint8_t* base, WsPtrs* out) const;
    // Device-pointer batch search on stream s (null: the borrowed workspace's
    // stream); waits for completion.
    void search_device(const float* d_q, size_t nq, size_t k, size_t nprobe, size_t pool,
                       int64_t* d_ids, float* d_dists, hipStream_t s);
    // The same over a caller-provided arena of `bytes` bytes (no allocation,
    // no statistics): queries go in chunks that fit it.
    void search_device_in(const float* d_q, size_t nq, size_t k, size_t nprobe, size_t pool,
                          int64_t* d_ids, float* d_dists, hipStream_t s, uint8_t* arena,
                          size_t bytes);
    void search_host(const float* q, size_t nq, size_t k, size_t nprobe, size_t pool,
                     int64_t* ids, float* dists);
    void probe_host(const float* q, size_t nq, size_t nprobe, uint32_t* lists);
    // search_host over given probe lists (probes[q*P..], P per query, every
    // list < L) instead of the coarse quantiser's: the file-backed searcher
    // probes with the full index's centroids and scans a batch index of the
    // probed lists.
    void search_host_probed(const float* q, size_t nq, size_t P, const uint32_t* probes, size_t k,
                            int64_t* ids, float* dists);
    void enable_filtering();
    void set_category(uint32_t doc_id, int cat);
    // search_with_filter for nq queries, query i restricted to category cats[i];
    // rows padded with (-1, +inf) like search_host.
    void search_filtered(const float* q, size_t nq, size_t k, const int* cats, int64_t* ids,
                         float* dists);
    vgpu_search_stats last_stats();
    void reconstruct(size_t idx, float* out) const;
    vgpu_memory_report memory_usage();

    // Borrow a workspace from the pool (a new one when all are in use).
    std::unique_ptr<SearchWs> take_ws();
    void give_ws(std::unique_ptr<SearchWs> ws);
    // Filtered search under OPQ rotates at most this many floats of residuals
    // per pass (queries go in chunks); settable for tests.
    size_t rres_limit = (size_t)1 << 28;

  private:
    // Every chunk of one search: coarse, select, scan, rerank and finish.
    // ws (may be null) supplies the profiling events and the pinned scalar
    // copy; *st receives the statistics when ws is given.
    // d_given (may be null): probe lists to use instead of the coarse step's.
    void run_search(const float* d_q, size_t nq, const SearchPlan& pl, const WsPtrs& w,
                    int64_t* d_ids, float* d_dists, hipStream_t s, SearchWs* ws,
                    vgpu_search_stats* st, const uint32_t* d_given = nullptr);
    // Normalise and probe nq queries into w.qn / w.qnorm / w.probe (P may be 0).
    // mid (may be null) is recorded between the scoring and the selection.
    // ordered: each row in ascending score order (the probe order of
    // search.rs:1602-1617); otherwise the same lists in no set order, which
    // is all a scan depends on.
    void coarse_probe(const float* d_q, size_t nq, size_t P, const SearchPlan& pl, const WsPtrs& w,
                      hipStream_t s, hipEvent_t mid, bool ordered = false);
    void kmeans_cosine(const std::vector<float>& x, size_t nt, size_t k, uint64_t seed,
                       size_t max_iter, std::vector<float>& cent);
    void assign_cosine(const float* d_x, const float* d_norms, size_t nx, const float* d_cent,
                       size_t k, float cmax, uint32_t* d_assign, hipStream_t s);
    void train_pq(const std::vector<float>& res, size_t nt, size_t Kc, uint64_t seed,
                  size_t max_iter);
    void train_opq(const std::vector<float>& res, size_t nt, uint64_t seed);
    // rotated residuals R (q_i - c_l) of nq queries x P slots into out[nq * P * d]
    void rotate_slots(const float* d_qn, size_t nq, size_t P, const uint32_t* d_lists, float* out,
                      hipStream_t s);
    void snapshot_list_masks();
    void refresh_categories(hipStream_t s);
};

struct FlatIndex {
    size_t d = 0;
    int metric = 0;
    size_t n = 0;
    hipStream_t stream = nullptr;
    hipEvent_t ev[4] = {};
    DevBuf<float> d_x, d_xnorm, w_q, w_dist, w_odist, w_qnorm;
    DevBuf<uint4> d_xb;  // bf16 hi/lo copy for the ranking kernel (d <= 128)
    DevBuf<uint64_t> w_partial, w_fbkeys;
    DevBuf<uint32_t> w_idx, w_flag, w_fb;
    DevBuf<int64_t> w_ids;
    DevBuf<unsigned int> w_overflow;
    std::vector<float> host;
    double xmax2 = 0.0;  // max ||x||^2
    float ms_gemm = 0.f, ms_total = 0.f;
    unsigned int fallbacks = 0;  // queries of the last search that took the exhaustive exact scan
    bool stale = false;  // a failed add could not restore the device copy of the n rows
    std::mutex mu;

    FlatIndex(size_t dim, int met);
    ~FlatIndex();
    // Appends count rows; on failure the index keeps its previous n rows.
    void add(const float* x, size_t count);
    void sync_device();  // device copy, norms and bf16 pack of host rows 0..n
    void search_device(const float* d_q, size_t nq, size_t k, int64_t* d_ids, float* d_dists,
                       hipStream_t s);
};

// A file descriptor closed with its owner (also when a constructor throws).
struct UniqueFd {
    int v = -1;
    UniqueFd() = default;
    UniqueFd(const UniqueFd&) = delete;
    UniqueFd& operator=(const UniqueFd&) = delete;
    ~UniqueFd();
};

// IVFPQFileSearcher (search.rs:247-262): routing metadata in memory, codes
// and raw vectors read from the snapshot directory per batch.  One batch at a
// time per handle (the reference's search takes &mut self).
struct FileIvfpq {
    size_t d = 0, L = 0, M = 0, K = 0, n = 0;
    vgpu_ivfpq_params params;
    std::string dir;
    std::vector<uint64_t> offsets;     // [L+1] list offsets into list_ids
    std::vector<uint32_t> list_ids;    // [n] snapshot vector index per list entry
    std::vector<uint32_t> doc_ids;     // [n]
    std::vector<float> centroids, codebooks;
    std::vector<uint64_t> lc_offsets;  // list_offsets.bin (bytes into list_codes.bin)
    UniqueFd fd_codes, fd_list_codes, fd_raw;
    std::unique_ptr<IvfpqIndex> meta;   // centroids only: the probe lists
    std::unique_ptr<IvfpqIndex> batch;  // the probed lists of the current batch
    hipStream_t stream = nullptr;
    DevBuf<float> d_vecs, d_q, d_qn, d_outd;
    DevBuf<uint32_t> d_rows, d_outrow;
    uint64_t io_bytes = 0, io_reads = 0;  // file reads of the last search
    std::mutex mu;

    FileIvfpq(size_t dim, const vgpu_ivfpq_params& p, const float* cent, size_t Lc, const float* cb,
              size_t Kc, const uint64_t* off, const uint32_t* lids, const uint32_t* dids, size_t nv,
              const float* rot, const std::string& directory, bool raw_present);
    ~FileIvfpq();
    void load_batch(const std::vector<uint32_t>& uni, std::vector<uint32_t>& members);
    void search(const float* q, size_t nq, size_t k, size_t nprobe, size_t pool, int64_t* ids,
                float* dists, vgpu_file_diagnostics* diag);
};

// Bytes of the allocation-free search's device scratch (one array per GPU).
#define NOALLOC_SCRATCH_BYTES ((size_t)64 << 20)
// The scratch array's device address on `device`, which must be current;
// looked up once per device (hipGetSymbolAddress) and kept.
uint8_t* noalloc_scratch(int device);
// Held across a whole allocation-free call on `device`, so calls from several
// threads (on any handles) take turns with the device's one array.
std::mutex& noalloc_call_mutex(int device);

// Host-side seeded sampling shared with the build (splitmix64 partial
// Fisher-Yates, ascending sample).
void sample_indices(size_t n, size_t sample, uint64_t seed, std::vector<uint32_t>& out);
void draw_distinct(size_t n, size_t count, uint64_t seed, std::vector<uint32_t>& out);
void normalize_row(const float* x, size_t d, float* out);
// Inverted lists from per-row list labels (insertion order inside a list);
// a label >= L raises VGPU_ERR_DEVICE.
void build_lists(const uint32_t* assign, size_t n, size_t L, std::vector<uint64_t>& offsets,
                 std::vector<uint32_t>& list_ids);
// Host cosine k-means update (float64 member means in row order, cast,
// re-normalised; empty keys keep their row) of cent[k * d]; a label >= k
// raises VGPU_ERR_DEVICE.
void centroid_update(const float* x, size_t n, size_t d, const uint32_t* assign, size_t k, float* cent);
// The orthogonal polar factor U V^T of M = U S V^T (d x d, row-major), in
// float64 by one-sided Jacobi, rounded to float32.
void polar_factor(const float* M, size_t d, float* R);

}  // namespace vgpu
