// extern "C" boundary: argument checks, exception -> status mapping and the
// thread-local error message.  Every entry point is declared in
// include/vicinity_gpu.h with the reference interface it replaces.
#include <algorithm>
#include <cmath>
#include <cstring>
#include <mutex>
#include <shared_mutex>
#include <string>

#include "vgpu_bounds.h"
#include "vgpu_runtime.h"

using vgpu::Error;
using vgpu::FlatIndex;
using vgpu::IvfpqIndex;

struct vgpu_ivfpq {
    IvfpqIndex* ix;
};
struct vgpu_flat {
    FlatIndex* fx;
};

namespace {

thread_local std::string g_last_error;

int fail(int code, const std::string& msg) {
    g_last_error = msg;
    return code;
}

template <typename F>
int guard(F&& f) {
    try {
        f();
        return VGPU_OK;
    } catch (const Error& e) {
        return fail(e.code, e.what());
    } catch (const std::bad_alloc&) {
        return fail(VGPU_ERR_OUT_OF_MEMORY, "host allocation failed");
    } catch (const std::exception& e) {
        return fail(VGPU_ERR_DEVICE, e.what());
    } catch (...) {
        return fail(VGPU_ERR_DEVICE, "unknown error");
    }
}

void need(bool ok, int code, const char* msg) {
    if (!ok) throw Error(code, msg);
}
void need(bool ok, int code, const std::string& msg) {
    if (!ok) throw Error(code, msg);
}

// Temporary device buffer for the per-kernel test entry points.
template <typename T>
struct Tmp : vgpu::DevBuf<T> {
    Tmp(const T* h, size_t n) { this->upload(h, n, nullptr); }
    explicit Tmp(size_t n) { this->reserve(n); }
};

}  // namespace

extern "C" {

const char* vgpu_last_error(void) { return g_last_error.c_str(); }

int vgpu_device_available(void) {
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || n <= 0) {
        (void)hipGetLastError();
        return 0;
    }
    hipDeviceProp_t prop;
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || hipGetDeviceProperties(&prop, dev) != hipSuccess) {
        (void)hipGetLastError();
        return 0;
    }
    return std::strncmp(prop.gcnArchName, "gfx950", 6) == 0 ? 1 : 0;
}

int vgpu_ivfpq_new(size_t dimension, const vgpu_ivfpq_params* params, vgpu_ivfpq** out) {
    return guard([&] {
        need(params && out, VGPU_ERR_INVALID_PARAMETER, "null argument");
        *out = nullptr;
        auto* h = new vgpu_ivfpq{nullptr};
        try {
            h->ix = new IvfpqIndex(dimension, *params);
        } catch (...) {
            delete h;
            throw;
        }
        *out = h;
    });
}

void vgpu_ivfpq_free(vgpu_ivfpq* h) {
    if (!h) return;
    delete h->ix;
    delete h;
}

int vgpu_ivfpq_add(vgpu_ivfpq* h, const uint32_t* doc_ids, const float* vectors, size_t n) {
    return guard([&] {
        need(h && (n == 0 || (doc_ids && vectors)), VGPU_ERR_INVALID_PARAMETER, "null argument");
        std::unique_lock<std::shared_mutex> lk(h->ix->mu);
        h->ix->add(doc_ids, vectors, n);
    });
}

int vgpu_ivfpq_build(vgpu_ivfpq* h, size_t training_sample_size, size_t kmeans_max_iter) {
    return guard([&] {
        need(h, VGPU_ERR_INVALID_PARAMETER, "null handle");
        std::unique_lock<std::shared_mutex> lk(h->ix->mu);
        h->ix->build(training_sample_size, kmeans_max_iter);
    });
}

int vgpu_ivfpq_load(vgpu_ivfpq* h, const float* centroids, size_t num_centroids,
                    const float* codebooks, size_t codebook_size, const uint64_t* list_offsets,
                    const uint32_t* list_ids, const uint8_t* codes, const uint32_t* doc_ids,
                    const float* vectors, size_t num_vectors) {
    return guard([&] {
        need(h && centroids && codebooks && list_offsets && (num_vectors == 0 || (list_ids && codes)),
             VGPU_ERR_INVALID_PARAMETER, "null argument");
        std::unique_lock<std::shared_mutex> lk(h->ix->mu);
        need(!h->ix->built, VGPU_ERR_ALREADY_BUILT, "IVF-PQ index is already built");
        h->ix->load(centroids, num_centroids, codebooks, codebook_size, list_offsets, list_ids, codes,
                    doc_ids, vectors, num_vectors);
    });
}

int vgpu_ivfpq_set_nprobe(vgpu_ivfpq* h, size_t nprobe) {
    return guard([&] {
        need(h, VGPU_ERR_INVALID_PARAMETER, "null handle");
        std::unique_lock<std::shared_mutex> lk(h->ix->mu);
        h->ix->params.nprobe = nprobe;
    });
}

int vgpu_ivfpq_set_mode(vgpu_ivfpq* h, int mode) {
    return guard([&] {
        need(h, VGPU_ERR_INVALID_PARAMETER, "null handle");
        need(mode == VGPU_MODE_FAST || mode == VGPU_MODE_EXACT, VGPU_ERR_INVALID_PARAMETER, "unknown mode");
        std::unique_lock<std::shared_mutex> lk(h->ix->mu);
        h->ix->mode = mode;
    });
}

int vgpu_ivfpq_set_profiling(vgpu_ivfpq* h, int enabled) {
    return guard([&] {
        need(h, VGPU_ERR_INVALID_PARAMETER, "null handle");
        std::unique_lock<std::shared_mutex> lk(h->ix->mu);
        need(enabled >= 0 && enabled <= 2, VGPU_ERR_INVALID_PARAMETER, "profiling level must be 0, 1 or 2");
        h->ix->profiling = enabled;
    });
}

int vgpu_ivfpq_compact(vgpu_ivfpq* h) {
    return guard([&] {
        need(h, VGPU_ERR_INVALID_PARAMETER, "null handle");
        std::unique_lock<std::shared_mutex> lk(h->ix->mu);
        need(h->ix->built, VGPU_ERR_INVALID_PARAMETER, "index must be built before compact");
        h->ix->vectors.clear();
        h->ix->vectors.shrink_to_fit();
        h->ix->has_vectors = false;
        h->ix->d_vectors.release();
        h->ix->dix.vectors = nullptr;
    });
}

int vgpu_ivfpq_get_info(const vgpu_ivfpq* h, vgpu_ivfpq_info* out) {
    return guard([&] {
        need(h && out, VGPU_ERR_INVALID_PARAMETER, "null argument");
        std::shared_lock<std::shared_mutex> lk(h->ix->mu);
        const IvfpqIndex& ix = *h->ix;
        out->dimension = ix.d;
        out->num_vectors = ix.n();
        out->num_clusters = ix.built ? ix.L : ix.params.num_clusters;
        out->nprobe = ix.params.nprobe;
        out->num_codebooks = ix.params.num_codebooks;
        out->codebook_size = ix.built ? ix.K : ix.params.codebook_size;
        out->subvector_dim = ix.params.num_codebooks ? ix.d / ix.params.num_codebooks : 0;
        out->built = ix.built ? 1 : 0;
        out->has_vectors = ix.has_vectors ? 1 : 0;
        out->mode = ix.mode;
    });
}

// search.rs:1188-1193: a query of the wrong length is DimensionMismatch.
static void check_dim(const IvfpqIndex& ix, size_t dim) {
    if (dim != ix.d)
        throw Error(VGPU_ERR_DIMENSION_MISMATCH, "dimension mismatch: query has " + std::to_string(dim) +
                                                     " values, index has " + std::to_string(ix.d));
}

int vgpu_ivfpq_search_batch(vgpu_ivfpq* h, const float* queries, size_t nq, size_t dim, size_t k,
                            size_t nprobe, size_t rerank_pool, int64_t* out_ids, float* out_dists) {
    return guard([&] {
        need(h && (nq == 0 || k == 0 || (queries && out_ids && out_dists)), VGPU_ERR_INVALID_PARAMETER,
             "null argument");
        std::shared_lock<std::shared_mutex> lk(h->ix->mu);
        need(h->ix->built, VGPU_ERR_NOT_BUILT, "IVF-PQ index: search before build");
        check_dim(*h->ix, dim);
        h->ix->search_host(queries, nq, k, nprobe, rerank_pool, out_ids, out_dists);
    });
}

int vgpu_ivfpq_search_batch_device(vgpu_ivfpq* h, const float* d_queries, size_t nq, size_t dim,
                                   size_t k, size_t nprobe, size_t rerank_pool, int64_t* d_out_ids,
                                   float* d_out_dists, void* stream) {
    return guard([&] {
        need(h && (nq == 0 || k == 0 || (d_queries && d_out_ids && d_out_dists)),
             VGPU_ERR_INVALID_PARAMETER, "null argument");
        std::shared_lock<std::shared_mutex> lk(h->ix->mu);
        need(h->ix->built, VGPU_ERR_NOT_BUILT, "IVF-PQ index: search before build");
        check_dim(*h->ix, dim);
        h->ix->search_device(d_queries, nq, k, nprobe, rerank_pool, d_out_ids, d_out_dists,
                             (hipStream_t)stream);
    });
}

int vgpu_ivfpq_search_batch_device_noalloc(vgpu_ivfpq* h, const float* d_queries, size_t nq, size_t dim,
                                           size_t k, size_t nprobe, size_t rerank_pool, int64_t* d_out_ids,
                                           float* d_out_dists, void* stream) {
    return guard([&] {
        need(h && (nq == 0 || k == 0 || (d_queries && d_out_ids && d_out_dists)),
             VGPU_ERR_INVALID_PARAMETER, "null argument");
        std::shared_lock<std::shared_mutex> lk(h->ix->mu);
        need(h->ix->built, VGPU_ERR_NOT_BUILT, "IVF-PQ index: search before build");
        check_dim(*h->ix, dim);
        if (nq == 0 || k == 0) return;
        uint8_t* scratch = vgpu::noalloc_scratch(h->ix->device);
        std::lock_guard<std::mutex> dev_lk(vgpu::noalloc_call_mutex(h->ix->device));
        h->ix->search_device_in(d_queries, nq, k, nprobe, rerank_pool, d_out_ids, d_out_dists,
                                (hipStream_t)stream, scratch, NOALLOC_SCRATCH_BYTES);
    });
}

// One query through the batch path; the result is truncated at the first
// padding entry (the reference returns fewer than k pairs in that case).
static int search_one(vgpu_ivfpq* h, const float* query, size_t dim, size_t k, size_t pool,
                      uint32_t* out_ids, float* out_dists, size_t* out_len) {
    return guard([&] {
        need(h && out_len && (k == 0 || (query && out_ids && out_dists)), VGPU_ERR_INVALID_PARAMETER,
             "null argument");
        std::shared_lock<std::shared_mutex> lk(h->ix->mu);
        *out_len = 0;
        need(h->ix->built, VGPU_ERR_NOT_BUILT, "IVF-PQ index: search before build");
        check_dim(*h->ix, dim);
        if (k == 0) return;
        std::vector<int64_t> ids(k);
        std::vector<float> dists(k);
        h->ix->search_host(query, 1, k, 0, pool, ids.data(), dists.data());
        size_t m = 0;
        while (m < k && ids[m] >= 0) {
            out_ids[m] = (uint32_t)ids[m];
            out_dists[m] = dists[m];
            m++;
        }
        *out_len = m;
    });
}

int vgpu_ivfpq_search(vgpu_ivfpq* h, const float* query, size_t dim, size_t k, uint32_t* out_ids,
                      float* out_dists, size_t* out_len) {
    return search_one(h, query, dim, k, 0, out_ids, out_dists, out_len);
}

int vgpu_ivfpq_search_reranked(vgpu_ivfpq* h, const float* query, size_t dim, size_t k, size_t pool,
                               uint32_t* out_ids, float* out_dists, size_t* out_len) {
    // search.rs:1144: pool = max(pool, k); a zero pool still reranks k.
    size_t p = pool < k ? k : pool;
    if (p == 0) p = 1;
    return search_one(h, query, dim, k, p, out_ids, out_dists, out_len);
}

int vgpu_ivfpq_last_stats(const vgpu_ivfpq* h, vgpu_search_stats* out) {
    return guard([&] {
        need(h && out, VGPU_ERR_INVALID_PARAMETER, "null argument");
        *out = h->ix->last_stats();
    });
}

int vgpu_ivfpq_enable_filtering(vgpu_ivfpq* h) {
    return guard([&] {
        need(h, VGPU_ERR_INVALID_PARAMETER, "null handle");
        std::unique_lock<std::shared_mutex> lk(h->ix->mu);
        h->ix->enable_filtering();
    });
}

int vgpu_ivfpq_set_category(vgpu_ivfpq* h, uint32_t doc_id, int64_t category) {
    return guard([&] {
        need(h, VGPU_ERR_INVALID_PARAMETER, "null handle");
        std::unique_lock<std::shared_mutex> lk(h->ix->mu);
        need(h->ix->filtering, VGPU_ERR_UNSUPPORTED,
             "filtered search: rebuild the index with IVFPQIndex::with_filtering()");
        need(category >= -1 && category <= 63, VGPU_ERR_INVALID_PARAMETER,
             "category ID " + std::to_string(category) + " exceeds bitmask limit of 63; use an integer in 0..63");
        h->ix->set_category(doc_id, (int)category);
    });
}

// One query; the result is truncated at the first padding entry.
int vgpu_ivfpq_search_filtered(vgpu_ivfpq* h, const float* query, size_t dim, size_t k, int64_t category,
                               uint32_t* out_ids, float* out_dists, size_t* out_len) {
    return guard([&] {
        need(h && out_len && (k == 0 || (query && out_ids && out_dists)), VGPU_ERR_INVALID_PARAMETER,
             "null argument");
        std::shared_lock<std::shared_mutex> lk(h->ix->mu);
        *out_len = 0;
        need(h->ix->built, VGPU_ERR_NOT_BUILT, "IVF-PQ index: search before build");
        check_dim(*h->ix, dim);
        need(h->ix->filtering, VGPU_ERR_INVALID_PARAMETER,
             "filter field doesn't match index filter field (None)");
        need(category >= 0 && category <= 63, VGPU_ERR_INVALID_PARAMETER,
             "category ID " + std::to_string(category) + " exceeds bitmask limit of 63");
        if (k == 0) return;
        std::vector<int64_t> ids(k);
        std::vector<float> dists(k);
        const int cat = (int)category;
        h->ix->search_filtered(query, 1, k, &cat, ids.data(), dists.data());
        size_t m = 0;
        while (m < k && ids[m] >= 0) {
            out_ids[m] = (uint32_t)ids[m];
            out_dists[m] = dists[m];
            m++;
        }
        *out_len = m;
    });
}

int vgpu_ivfpq_search_filtered_batch(vgpu_ivfpq* h, const float* queries, size_t nq, size_t dim, size_t k,
                                     const int64_t* categories, int64_t* out_ids, float* out_dists) {
    return guard([&] {
        need(h && (nq == 0 || k == 0 || (queries && categories && out_ids && out_dists)),
             VGPU_ERR_INVALID_PARAMETER, "null argument");
        std::shared_lock<std::shared_mutex> lk(h->ix->mu);
        need(h->ix->built, VGPU_ERR_NOT_BUILT, "IVF-PQ index: search before build");
        check_dim(*h->ix, dim);
        need(h->ix->filtering, VGPU_ERR_INVALID_PARAMETER,
             "filter field doesn't match index filter field (None)");
        std::vector<int> cats(nq);
        for (size_t i = 0; i < nq; i++) {
            need(categories[i] >= 0 && categories[i] <= 63, VGPU_ERR_INVALID_PARAMETER,
                 "category ID " + std::to_string(categories[i]) + " exceeds bitmask limit of 63");
            cats[i] = (int)categories[i];
        }
        if (nq == 0 || k == 0) return;
        h->ix->search_filtered(queries, nq, k, cats.data(), out_ids, out_dists);
    });
}

int vgpu_ivfpq_get_list_masks(const vgpu_ivfpq* h, uint64_t* masks, size_t L) {
    return guard([&] {
        need(h && (L == 0 || masks), VGPU_ERR_INVALID_PARAMETER, "null argument");
        std::shared_lock<std::shared_mutex> lk(h->ix->mu);
        need(h->ix->built, VGPU_ERR_NOT_BUILT, "IVF-PQ index: list bitmasks before build");
        need(L == h->ix->L, VGPU_ERR_INVALID_PARAMETER, "list count mismatch");
        for (size_t l = 0; l < L; l++) masks[l] = l < h->ix->list_mask.size() ? h->ix->list_mask[l] : 0ull;
    });
}

int vgpu_ivfpq_set_list_masks(vgpu_ivfpq* h, const uint64_t* masks, size_t L) {
    return guard([&] {
        need(h && (L == 0 || masks), VGPU_ERR_INVALID_PARAMETER, "null argument");
        std::unique_lock<std::shared_mutex> lk(h->ix->mu);
        need(h->ix->built, VGPU_ERR_NOT_BUILT, "IVF-PQ index: list bitmasks before build");
        need(L == h->ix->L, VGPU_ERR_INVALID_PARAMETER, "list count mismatch");
        h->ix->list_mask.assign(masks, masks + L);
    });
}

int vgpu_ivfpq_get_rotation(const vgpu_ivfpq* h, float* R, size_t len, int* present) {
    return guard([&] {
        need(h && present, VGPU_ERR_INVALID_PARAMETER, "null argument");
        std::shared_lock<std::shared_mutex> lk(h->ix->mu);
        const auto& rot = h->ix->rotation;
        *present = rot.empty() ? 0 : 1;
        if (rot.empty()) return;
        need(R && len == rot.size(), VGPU_ERR_INVALID_PARAMETER, "rotation buffer must hold dim * dim floats");
        std::copy(rot.begin(), rot.end(), R);
    });
}

int vgpu_ivfpq_set_rotation(vgpu_ivfpq* h, const float* R, size_t len) {
    return guard([&] {
        need(h, VGPU_ERR_INVALID_PARAMETER, "null argument");
        std::unique_lock<std::shared_mutex> lk(h->ix->mu);
        need(!R || len == h->ix->d * h->ix->d, VGPU_ERR_INVALID_PARAMETER, "rotation must hold dim * dim floats");
        h->ix->set_rotation(R);
    });
}

int vgpu_ivfpq_probe_batch(vgpu_ivfpq* h, const float* queries, size_t nq, size_t dim, size_t nprobe,
                           uint32_t* lists, size_t* out_p) {
    return guard([&] {
        need(h && out_p && (nq == 0 || (queries && lists)), VGPU_ERR_INVALID_PARAMETER, "null argument");
        std::shared_lock<std::shared_mutex> lk(h->ix->mu);
        need(h->ix->built, VGPU_ERR_NOT_BUILT, "IVF-PQ index: probe before build");
        check_dim(*h->ix, dim);
        *out_p = std::min(nprobe, h->ix->L);
        for (size_t i = 0; i < nq * h->ix->d; i++)
            need(std::isfinite(queries[i]), VGPU_ERR_INVALID_PARAMETER, "query contains a non-finite value");
        h->ix->probe_host(queries, nq, nprobe, lists);
    });
}

int vgpu_ivfpq_export(const vgpu_ivfpq* h, float* centroids, float* codebooks, uint64_t* list_offsets,
                      uint32_t* list_ids, uint8_t* codes, uint32_t* doc_ids, float* vectors) {
    return guard([&] {
        need(h, VGPU_ERR_INVALID_PARAMETER, "null handle");
        std::shared_lock<std::shared_mutex> lk(h->ix->mu);
        const IvfpqIndex& ix = *h->ix;
        need(ix.built, VGPU_ERR_NOT_BUILT, "IVF-PQ index: export before build");
        auto cp = [](void* dst, const void* src, size_t bytes) {
            if (dst && bytes) std::memcpy(dst, src, bytes);
        };
        cp(centroids, ix.centroids.data(), ix.centroids.size() * sizeof(float));
        cp(codebooks, ix.codebooks.data(), ix.codebooks.size() * sizeof(float));
        cp(list_offsets, ix.offsets.data(), ix.offsets.size() * sizeof(uint64_t));
        cp(list_ids, ix.list_ids.data(), ix.list_ids.size() * sizeof(uint32_t));
        cp(codes, ix.codes.data(), ix.codes.size());
        cp(doc_ids, ix.doc_ids.data(), ix.doc_ids.size() * sizeof(uint32_t));
        if (vectors) {
            need(ix.has_vectors, VGPU_ERR_UNSUPPORTED, "raw vectors were dropped by compact()");
            cp(vectors, ix.vectors.data(), ix.vectors.size() * sizeof(float));
        }
    });
}

int vgpu_ivfpq_reconstruct(const vgpu_ivfpq* h, size_t idx, float* out, size_t len) {
    return guard([&] {
        need(h && out, VGPU_ERR_INVALID_PARAMETER, "null argument");
        std::shared_lock<std::shared_mutex> lk(h->ix->mu);
        need(len >= h->ix->d, VGPU_ERR_INVALID_PARAMETER, "output shorter than the dimension");
        h->ix->reconstruct(idx, out);
    });
}

int vgpu_ivfpq_memory_usage(const vgpu_ivfpq* h, vgpu_memory_report* out) {
    return guard([&] {
        need(h && out, VGPU_ERR_INVALID_PARAMETER, "null argument");
        std::shared_lock<std::shared_mutex> lk(h->ix->mu);
        *out = h->ix->memory_usage();
    });
}

/* ---- flat ---------------------------------------------------------------- */

int vgpu_flat_new(size_t dimension, int metric, vgpu_flat** out) {
    return guard([&] {
        need(out != nullptr, VGPU_ERR_INVALID_PARAMETER, "null argument");
        *out = nullptr;
        auto* h = new vgpu_flat{nullptr};
        try {
            h->fx = new FlatIndex(dimension, metric);
        } catch (...) {
            delete h;
            throw;
        }
        *out = h;
    });
}

void vgpu_flat_free(vgpu_flat* h) {
    if (!h) return;
    delete h->fx;
    delete h;
}

int vgpu_flat_add(vgpu_flat* h, const float* vectors, size_t n) {
    return guard([&] {
        need(h && (n == 0 || vectors), VGPU_ERR_INVALID_PARAMETER, "null argument");
        std::lock_guard<std::mutex> lk(h->fx->mu);
        h->fx->add(vectors, n);
    });
}

int vgpu_flat_search_batch(vgpu_flat* h, const float* queries, size_t nq, size_t dim, size_t k,
                           int64_t* out_ids, float* out_dists) {
    return guard([&] {
        need(h && (nq == 0 || k == 0 || (queries && out_ids && out_dists)), VGPU_ERR_INVALID_PARAMETER,
             "null argument");
        std::lock_guard<std::mutex> lk(h->fx->mu);
        FlatIndex& fx = *h->fx;
        need(dim == fx.d, VGPU_ERR_DIMENSION_MISMATCH, "dimension mismatch");
        if (nq == 0 || k == 0) return;
        for (size_t i = 0; i < nq * fx.d; i++)
            need(std::isfinite(queries[i]), VGPU_ERR_INVALID_PARAMETER, "query contains a non-finite value");
        fx.w_q.upload(queries, nq * fx.d, fx.stream);
        fx.w_ids.reserve(nq * k);
        fx.w_odist.reserve(nq * k);
        fx.search_device(fx.w_q.p, nq, k, fx.w_ids.p, fx.w_odist.p, fx.stream);
        VGPU_HIP(hipMemcpyAsync(out_ids, fx.w_ids.p, nq * k * sizeof(int64_t), hipMemcpyDeviceToHost, fx.stream));
        VGPU_HIP(hipMemcpyAsync(out_dists, fx.w_odist.p, nq * k * sizeof(float), hipMemcpyDeviceToHost, fx.stream));
        VGPU_HIP(hipStreamSynchronize(fx.stream));
    });
}

int vgpu_flat_search_batch_device(vgpu_flat* h, const float* d_queries, size_t nq, size_t dim,
                                  size_t k, int64_t* d_out_ids, float* d_out_dists, void* stream) {
    return guard([&] {
        need(h && (nq == 0 || k == 0 || (d_queries && d_out_ids && d_out_dists)),
             VGPU_ERR_INVALID_PARAMETER, "null argument");
        std::lock_guard<std::mutex> lk(h->fx->mu);
        need(dim == h->fx->d, VGPU_ERR_DIMENSION_MISMATCH, "dimension mismatch");
        h->fx->search_device(d_queries, nq, k, d_out_ids, d_out_dists, (hipStream_t)stream);
        VGPU_HIP(hipStreamSynchronize(stream ? (hipStream_t)stream : h->fx->stream));
    });
}

int vgpu_flat_last_ms(const vgpu_flat* h, float* ms_gemm, float* ms_total) {
    return guard([&] {
        need(h, VGPU_ERR_INVALID_PARAMETER, "null handle");
        std::lock_guard<std::mutex> lk(h->fx->mu);
        if (ms_gemm) *ms_gemm = h->fx->ms_gemm;
        if (ms_total) *ms_total = h->fx->ms_total;
    });
}

int vgpu_flat_last_fallbacks(const vgpu_flat* h, uint32_t* queries) {
    return guard([&] {
        need(h && queries, VGPU_ERR_INVALID_PARAMETER, "null argument");
        std::lock_guard<std::mutex> lk(h->fx->mu);
        *queries = h->fx->fallbacks;
    });
}

/* ---- per-kernel test entry points ---------------------------------------- */

int vgpu_test_host_lists(const uint32_t* assign, size_t n, size_t L, uint64_t* offsets, uint32_t* list_ids) {
    return guard([&] {
        need((n == 0 || (assign && list_ids)) && offsets && L, VGPU_ERR_INVALID_PARAMETER, "bad argument");
        std::vector<uint64_t> off;
        std::vector<uint32_t> ids;
        vgpu::build_lists(assign, n, L, off, ids);
        std::copy(off.begin(), off.end(), offsets);
        std::copy(ids.begin(), ids.end(), list_ids);
    });
}

int vgpu_test_host_centroid_update(const float* x, size_t n, size_t d, const uint32_t* assign, size_t k,
                                   float* centroids) {
    return guard([&] {
        need((n == 0 || (x && assign)) && centroids && d && k, VGPU_ERR_INVALID_PARAMETER, "bad argument");
        vgpu::centroid_update(x, n, d, assign, k, centroids);
    });
}

int vgpu_test_polar_factor(const float* m, size_t d, float* r) {
    return guard([&] {
        need(m && r && d, VGPU_ERR_INVALID_PARAMETER, "bad argument");
        vgpu::polar_factor(m, d, r);
    });
}

struct vgpu_ivfpq_file {
    vgpu::FileIvfpq* fx;
};

int vgpu_ivfpq_file_open(size_t dimension, const vgpu_ivfpq_params* params, const float* centroids,
                         size_t num_centroids, const float* codebooks, size_t codebook_size,
                         const uint64_t* list_offsets, const uint32_t* list_ids, const uint32_t* doc_ids,
                         size_t num_vectors, const float* rotation, const char* dir, int raw_vectors_present,
                         vgpu_ivfpq_file** out) {
    return guard([&] {
        need(params && centroids && codebooks && list_offsets && dir && out, VGPU_ERR_INVALID_PARAMETER,
             "null argument");
        *out = nullptr;
        auto* h = new vgpu_ivfpq_file{nullptr};
        try {
            h->fx = new vgpu::FileIvfpq(dimension, *params, centroids, num_centroids, codebooks, codebook_size,
                                        list_offsets, list_ids, doc_ids, num_vectors, rotation, dir,
                                        raw_vectors_present != 0);
        } catch (...) {
            delete h;
            throw;
        }
        *out = h;
    });
}

void vgpu_ivfpq_file_free(vgpu_ivfpq_file* h) {
    if (!h) return;
    delete h->fx;
    delete h;
}

int vgpu_ivfpq_file_set_nprobe(vgpu_ivfpq_file* h, size_t nprobe) {
    return guard([&] {
        need(h, VGPU_ERR_INVALID_PARAMETER, "null handle");
        std::lock_guard<std::mutex> lk(h->fx->mu);
        h->fx->params.nprobe = nprobe;
    });
}

int vgpu_ivfpq_file_search_batch(vgpu_ivfpq_file* h, const float* queries, size_t nq, size_t dim, size_t k,
                                 size_t nprobe, size_t rerank_pool, int64_t* out_ids, float* out_dists,
                                 vgpu_file_diagnostics* diag) {
    return guard([&] {
        need(h && (nq == 0 || queries) && (nq * k == 0 || (out_ids && out_dists)), VGPU_ERR_INVALID_PARAMETER,
             "null argument");
        std::lock_guard<std::mutex> lk(h->fx->mu);
        need(dim == h->fx->d, VGPU_ERR_DIMENSION_MISMATCH, "query dimension does not match the index");
        h->fx->search(queries, nq, k, nprobe, rerank_pool, out_ids, out_dists, diag);
    });
}

int vgpu_ivfpq_file_last_io(const vgpu_ivfpq_file* h, uint64_t* reads, uint64_t* bytes) {
    return guard([&] {
        need(h && reads && bytes, VGPU_ERR_INVALID_PARAMETER, "null argument");
        std::lock_guard<std::mutex> lk(h->fx->mu);
        *reads = h->fx->io_reads;
        *bytes = h->fx->io_bytes;
    });
}

int vgpu_test_bound_fast_tau(size_t d, size_t M, size_t ds, float qn, float cmax, float rmax,
                             float t0max, float* out) {
    return guard([&] {
        need(out && d && M && ds, VGPU_ERR_INVALID_PARAMETER, "bad argument");
        *out = vgpu::fast_tau((int)d, (int)M, (int)ds, qn, cmax, rmax, t0max);
    });
}

int vgpu_test_bound_coarse(size_t d, float qn, float cmax, float* out_bf16x3, float* out_fp32) {
    return guard([&] {
        need(out_bf16x3 && out_fp32 && d, VGPU_ERR_INVALID_PARAMETER, "bad argument");
        *out_bf16x3 = vgpu::coarse_eps_bf16((int)d, qn, cmax);
        *out_fp32 = vgpu::coarse_tau((int)d, qn, cmax);
    });
}

int vgpu_test_bound_flat(size_t d, int metric, float qn, float xn, int ib, float* out) {
    return guard([&] {
        need(out && d && (metric == 0 || metric == 1) && ib >= 0 && ib < 24,
             VGPU_ERR_INVALID_PARAMETER, "bad argument");
        *out = vgpu::flat_bf16_tau((int)d, metric, qn, xn, ib);
    });
}

int vgpu_test_fail_device_allocations(size_t after, size_t count) {
    return guard([&] { vgpu::arm_alloc_failures((long long)after, (long long)count); });
}

int vgpu_test_set_rres_limit(vgpu_ivfpq* h, size_t floats) {
    return guard([&] {
        need(h && floats, VGPU_ERR_INVALID_PARAMETER, "bad argument");
        std::unique_lock<std::shared_mutex> lk(h->ix->mu);
        h->ix->rres_limit = floats;
    });
}

int vgpu_test_adc_tables(const float* codebooks, size_t M, size_t K, size_t ds, const float* residuals,
                         size_t nr, float* tables) {
    return guard([&] {
        need(codebooks && residuals && tables && M && K && ds, VGPU_ERR_INVALID_PARAMETER, "bad argument");
        Tmp<float> cb(codebooks, M * K * ds), r(residuals, nr * M * ds), t(nr * M * K);
        vgpu::launch_adc_tables(cb.p, (int)M, (int)K, (int)ds, r.p, (int)nr, t.p, nullptr);
        VGPU_HIP(hipGetLastError());
        VGPU_HIP(hipMemcpy(tables, t.p, nr * M * K * sizeof(float), hipMemcpyDeviceToHost));
    });
}

int vgpu_test_pq_encode(const float* codebooks, size_t M, size_t K, size_t ds, const float* x, size_t n,
                        uint8_t* codes) {
    return guard([&] {
        need(codebooks && x && codes && M && K && K <= 256 && ds, VGPU_ERR_INVALID_PARAMETER, "bad argument");
        Tmp<float> cb(codebooks, M * K * ds), xv(x, n * M * ds);
        Tmp<uint8_t> c(n * M);
        vgpu::launch_encode(xv.p, (int)n, (int)(M * ds), nullptr, nullptr, cb.p, (int)M, (int)K, (int)ds,
                            c.p, nullptr);
        VGPU_HIP(hipGetLastError());
        VGPU_HIP(hipMemcpy(codes, c.p, n * M, hipMemcpyDeviceToHost));
    });
}

int vgpu_test_normalize(const float* x, size_t n, size_t d, float* out) {
    return guard([&] {
        need(x && out && d, VGPU_ERR_INVALID_PARAMETER, "bad argument");
        Tmp<float> xv(x, n * d), o(n * d), nr(n);
        vgpu::launch_normalize(xv.p, o.p, nr.p, (int)n, (int)d, nullptr);
        VGPU_HIP(hipGetLastError());
        VGPU_HIP(hipMemcpy(out, o.p, n * d * sizeof(float), hipMemcpyDeviceToHost));
    });
}

int vgpu_test_fastscan(const uint8_t* packed, size_t n, size_t M, const float* lut, float* out) {
    return guard([&] {
        need(packed && lut && out && M, VGPU_ERR_INVALID_PARAMETER, "bad argument");
        need(M <= 257, VGPU_ERR_INVALID_PARAMETER,
             "FastScan accumulates LUT terms in u16: more than 257 codebooks would overflow");
        size_t bytes = ((n + 31) / 32) * 16 * M;
        Tmp<uint8_t> p(packed, bytes ? bytes : 1);
        Tmp<float> l(lut, M * 16), o(n ? n : 1);
        vgpu::launch_fastscan_test(p.p, (int)n, (int)M, l.p, o.p, nullptr);
        VGPU_HIP(hipGetLastError());
        VGPU_HIP(hipMemcpy(out, o.p, n * sizeof(float), hipMemcpyDeviceToHost));
    });
}

int vgpu_test_coarse_dots(const float* q, size_t nq, const float* c, size_t L, size_t d, float* out) {
    return guard([&] {
        need(q && c && out && d, VGPU_ERR_INVALID_PARAMETER, "bad argument");
        Tmp<float> qv(q, nq * d), cv(c, L * d), o(nq * L);
        vgpu::launch_coarse_dots(qv.p, cv.p, o.p, (int)nq, (int)L, (int)d, nullptr);
        VGPU_HIP(hipGetLastError());
        VGPU_HIP(hipMemcpy(out, o.p, nq * L * sizeof(float), hipMemcpyDeviceToHost));
    });
}

int vgpu_test_coarse_dots_bf16x3(const float* q, size_t nq, const float* c, size_t L, size_t d,
                                 float* out) {
    return guard([&] {
        need(q && c && out && d && L, VGPU_ERR_INVALID_PARAMETER, "bad argument");
        need(d <= 128, VGPU_ERR_INVALID_PARAMETER, "the bf16x3 coarse kernel takes d <= 128");
        Tmp<float> qv(q, nq * d), cv(c, L * d), o(nq * L ? nq * L : 1);
        vgpu::DevBuf<uint4> cb;
        cb.reserve(vgpu::coarse_bf16_pack_chunks((int)L, (int)d));
        vgpu::launch_coarse_bf16_pack(cv.p, (int)L, (int)d, cb.p, nullptr);
        vgpu::launch_coarse_bf16x3_dots(qv.p, (int)nq, (int)d, cb.p, (int)L, o.p, nullptr);
        VGPU_HIP(hipGetLastError());
        VGPU_HIP(hipMemcpy(out, o.p, nq * L * sizeof(float), hipMemcpyDeviceToHost));
    });
}

}  // extern "C"
