// Host runtime: device buffers, HIP error mapping and the IVF-PQ / flat index
// objects behind the C ABI.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <mutex>
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
    // Grow-only allocation (contents are not preserved on growth).
    void reserve(size_t count) {
        if (count <= n && p) return;
        release();
        size_t bytes = (count ? count : 1) * sizeof(T);
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

// A built IVF-PQ index.  Mirrors the state of IVFPQIndex
// (src/ivf_pq/search.rs:212-239): the raw normalised vectors and doc ids on
// the host, the search arrays resident in HBM.
struct IvfpqIndex {
    size_t d = 0;
    vgpu_ivfpq_params params{};
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

    hipStream_t stream = nullptr;
    hipEvent_t ev[8] = {};
    std::vector<hipEvent_t> sev;  // scan-only timing: two per chunk
    DevBuf<float> d_centroids, d_codebooks, d_bias, d_vectors, d_rotation;
    DevBuf<uint4> d_cb16, w_cb16;  // bf16 hi/lo centroid copies (search index, build workspace)
    DevBuf<uint32_t> w_cand, w_cand_n;  // fused coarse candidates
    DevBuf<uint32_t> d_offsets, d_list_ids, d_doc_ids, d_pack_off;
    DevBuf<uint8_t> d_codes, d_packed, d_tblocks;
    DevBuf<uint32_t> d_tblk_off;
    DevIndex dix;

    // search workspace
    DevBuf<float> w_q, w_qn, w_qnorm, w_dots, w_dist, w_dist2, w_odist;
    DevBuf<float> w_rres;  // OPQ: rotated residual of each (query, slot)
    DevBuf<uint32_t> w_probe, w_vidx, w_vidx2, w_qstat, w_flag_list;
    DevBuf<uint32_t> w_cflag_list, w_cflag_count;  // coarse selection fallback list
    DevBuf<int64_t> w_ids;
    DevBuf<unsigned long long> w_scal;           // per-call device scalars (see search_device)
    unsigned long long* h_scal = nullptr;        // pinned host copy of w_scal
    DevBuf<unsigned int> w_overflow;
    vgpu_search_stats stats{};
    std::mutex mu;

    // search_with_filter state (search.rs:236-238): the category each document
    // carries in the filter field, per-list bitmasks taken when the lists are
    // built (search.rs:626-648), and device copies refreshed on demand.
    bool filtering = false;
    std::unordered_map<uint32_t, int> doc_cat;  // doc id -> 0..63, or -1 (metadata without the field)
    std::vector<uint64_t> list_mask;            // [L]
    std::vector<uint32_t> list_cat_n;           // [L*64] entries per (list, category), current metadata
    bool cat_dirty = true;
    DevBuf<uint8_t> d_ecat, w_want;  // category of each list-major entry (0xff: none); per query

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
    // Device-pointer batch search on stream s (s may be null = own stream).
    void search_device(const float* d_q, size_t nq, size_t k, size_t nprobe, size_t pool,
                       int64_t* d_ids, float* d_dists, hipStream_t s);
    void search_host(const float* q, size_t nq, size_t k, size_t nprobe, size_t pool,
                     int64_t* ids, float* dists);
    void probe_host(const float* q, size_t nq, size_t nprobe, uint32_t* lists);
    void enable_filtering();
    void set_category(uint32_t doc_id, int cat);
    // search_with_filter for nq queries, query i restricted to category cats[i];
    // rows padded with (-1, +inf) like search_host.
    void search_filtered(const float* q, size_t nq, size_t k, const int* cats, int64_t* ids,
                         float* dists);

  private:
    void kmeans_cosine(const std::vector<float>& x, size_t nt, size_t k, uint64_t seed,
                       size_t max_iter, std::vector<float>& cent);
    void assign_cosine(const float* d_x, const float* d_norms, size_t nx, const float* d_cent,
                       size_t k, float cmax, uint32_t* d_assign, hipStream_t s);
    void train_pq(const std::vector<float>& res, size_t nt, size_t Kc, uint64_t seed,
                  size_t max_iter);
    void train_opq(const std::vector<float>& res, size_t nt, uint64_t seed);
    // rotated residuals R (q_i - c_l) of nq queries x P slots into w_rres
    const float* rotate_slots(const float* d_qn, size_t nq, size_t P, const uint32_t* d_lists,
                              hipStream_t s);
    void snapshot_list_masks();
    void refresh_categories();
};

struct FlatIndex {
    size_t d = 0;
    int metric = 0;
    size_t n = 0;
    hipStream_t stream = nullptr;
    hipEvent_t ev[4] = {};
    DevBuf<float> d_x, d_xnorm, w_q, w_dist, w_odist, w_qnorm;
    DevBuf<uint64_t> w_partial;
    DevBuf<uint32_t> w_idx;
    DevBuf<int64_t> w_ids;
    DevBuf<unsigned int> w_overflow;
    std::vector<float> host;
    double xmax2 = 0.0;  // max ||x||^2
    float ms_gemm = 0.f, ms_total = 0.f;
    std::mutex mu;

    FlatIndex(size_t dim, int met);
    ~FlatIndex();
    void add(const float* x, size_t count);
    void search_device(const float* d_q, size_t nq, size_t k, int64_t* d_ids, float* d_dists,
                       hipStream_t s);
};

// Host-side seeded sampling shared with the build (splitmix64 partial
// Fisher-Yates, ascending sample).
void sample_indices(size_t n, size_t sample, uint64_t seed, std::vector<uint32_t>& out);
void draw_distinct(size_t n, size_t count, uint64_t seed, std::vector<uint32_t>& out);
void normalize_row(const float* x, size_t d, float* out);
// The orthogonal polar factor U V^T of M = U S V^T (d x d, row-major), in
// float64 by one-sided Jacobi, rounded to float32.
void polar_factor(const float* M, size_t d, float* R);

}  // namespace vgpu
