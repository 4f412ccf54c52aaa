// IVF-PQ index object: insert, GPU-assisted build, HBM residency, and the
// batched search pipeline.
//
// Reference: IVFPQIndex src/ivf_pq/search.rs:212-239 (state), add_slice
// :488-512, build_with_training_config :546-787, build_scan_caches :816-848,
// search :1087-1093, search_reranked :1117-1158, search_approx_internal_observed
// :1175-1391; batch shape src/python.rs:744-793.
#include <algorithm>
#include <atomic>
#include <cmath>
#include <cstring>
#include <numeric>
#include <type_traits>
#include <unordered_map>

#include "vgpu_runtime.h"

namespace vgpu {

void ensure_dyn_lds(const void* kernel, size_t bytes) {
    static std::mutex mu;
    static std::unordered_map<const void*, size_t> set;
    std::lock_guard<std::mutex> lock(mu);
    size_t& cur = set[kernel];
    if (bytes <= cur) return;
    if (hipFuncSetAttribute(kernel, hipFuncAttributeMaxDynamicSharedMemorySize, (int)bytes) == hipSuccess)
        cur = bytes;
    else
        (void)hipGetLastError();
}

void hip_check(hipError_t e, const char* what) {
    if (e == hipSuccess) return;
    (void)hipGetLastError();
    int code = (e == hipErrorOutOfMemory || e == hipErrorMemoryAllocation) ? VGPU_ERR_OUT_OF_MEMORY
                                                                           : VGPU_ERR_DEVICE;
    throw Error(code, std::string(what) + ": " + hipGetErrorString(e));
}

namespace {
std::atomic<long long> g_fail_after{0}, g_fail_count{0};
}

void arm_alloc_failures(long long after, long long count) {
    g_fail_count.store(0);
    g_fail_after.store(after < 0 ? 0 : after);
    g_fail_count.store(count < 0 ? 0 : count);
}

bool alloc_should_fail() {
    if (g_fail_count.load(std::memory_order_relaxed) <= 0) return false;
    long long a = g_fail_after.load();
    while (a > 0)
        if (g_fail_after.compare_exchange_weak(a, a - 1)) return false;
    long long c = g_fail_count.load();
    while (c > 0)
        if (g_fail_count.compare_exchange_weak(c, c - 1)) return true;
    return false;
}

// splitmix64 (Steele, Lea, Flood 2014): the seeded stream of the training
// sample and of the k-means initial centroids.
static inline uint64_t splitmix64(uint64_t& s) {
    uint64_t z = (s += 0x9E3779B97F4A7C15ull);
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

static inline size_t bounded(uint64_t& s, size_t n) {
    return (size_t)(((unsigned __int128)splitmix64(s) * (unsigned __int128)n) >> 64);
}

void draw_distinct(size_t n, size_t count, uint64_t seed, std::vector<uint32_t>& out) {
    std::vector<uint32_t> perm(n);
    std::iota(perm.begin(), perm.end(), 0u);
    uint64_t s = seed;
    out.resize(count);
    for (size_t i = 0; i < count; i++) {
        size_t j = i + bounded(s, n - i);
        std::swap(perm[i], perm[j]);
        out[i] = perm[i];
    }
}

void sample_indices(size_t n, size_t sample, uint64_t seed, std::vector<uint32_t>& out) {
    if (sample == 0 || sample >= n) {
        out.resize(n);
        std::iota(out.begin(), out.end(), 0u);
        return;
    }
    draw_distinct(n, sample, seed, out);
    std::sort(out.begin(), out.end());
}

// search.rs:55-62 / :503-508: sum of squares in order, sqrt, x / norm when
// norm > 1e-10 (this file is compiled with -ffp-contract=off).
void normalize_row(const float* x, size_t d, float* out) {
    float s = 0.0f;
    for (size_t i = 0; i < d; i++) s += x[i] * x[i];
    float norm = std::sqrt(s);
    if (norm > 1e-10f) {
        for (size_t i = 0; i < d; i++) out[i] = x[i] / norm;
    } else if (out != x) {
        std::memcpy(out, x, d * sizeof(float));
    }
}

// Labels read back from the device index host arrays: one outside 0..L-1
// means the device returned garbage, reported as a device error instead of
// being used as an index.
template <typename T>
static void check_labels(const T* labels, size_t n, size_t stride, size_t L, const char* what) {
    for (size_t i = 0; i < n; i++)
        if ((size_t)labels[i * stride] >= L)
            throw Error(VGPU_ERR_DEVICE, std::string(what) + ": row " + std::to_string(i) + " has label " +
                                             std::to_string((size_t)labels[i * stride]) + ", outside 0.." +
                                             std::to_string(L - 1));
}

// Inverted lists from list labels (search.rs:624-657): list l holds the rows
// labelled l in insertion order; offsets[L + 1], list_ids[n].
void build_lists(const uint32_t* assign, size_t n, size_t L, std::vector<uint64_t>& offsets,
                 std::vector<uint32_t>& list_ids) {
    check_labels(assign, n, 1, L, "list assignment");
    offsets.assign(L + 1, 0);
    for (size_t i = 0; i < n; i++) offsets[assign[i] + 1]++;
    for (size_t l = 0; l < L; l++) offsets[l + 1] += offsets[l];
    list_ids.resize(n);
    std::vector<uint64_t> fill(offsets.begin(), offsets.end() - 1);
    for (size_t i = 0; i < n; i++) list_ids[fill[assign[i]]++] = (uint32_t)i;
}

// Lloyd update on the host (rows wider than the update kernel's 256
// floats): every non-empty key becomes the float64 mean of its members in
// row order, cast to float, re-normalised when `normalize`; empty keys keep
// their row.  Row i's slice is x[i * ld + off .. + w), its label
// labels[i * lstride]; out[k * w].
template <typename T>
static void host_mean_update(const float* x, size_t n, size_t ld, size_t off, size_t w, const T* labels,
                             size_t lstride, size_t k, bool normalize, float* out) {
    check_labels(labels, n, lstride, k, "k-means labels");
    std::vector<double> sums(k * w, 0.0);
    std::vector<uint64_t> counts(k, 0);
    for (size_t i = 0; i < n; i++) {
        const size_t c = (size_t)labels[i * lstride];
        double* sc = &sums[c * w];
        const float* xi = &x[i * ld + off];
        for (size_t j = 0; j < w; j++) sc[j] += (double)xi[j];
        counts[c]++;
    }
    for (size_t c = 0; c < k; c++) {
        if (!counts[c]) continue;
        float* cc = &out[c * w];
        for (size_t j = 0; j < w; j++) cc[j] = (float)(sums[c * w + j] / (double)counts[c]);
        if (normalize) normalize_row(cc, w, cc);
    }
}

void centroid_update(const float* x, size_t n, size_t d, const uint32_t* assign, size_t k, float* cent) {
    host_mean_update(x, n, d, 0, d, assign, 1, k, true, cent);
}

static float row_norm_bound(const float* x, size_t d) {
    double s = 0.0;
    for (size_t i = 0; i < d; i++) s += (double)x[i] * (double)x[i];
    return (float)(std::sqrt(s) * 1.0001 + 1e-30);
}

IvfpqIndex::IvfpqIndex(size_t dim, const vgpu_ivfpq_params& p) : d(dim), params(p) {
    if (dim == 0) throw Error(VGPU_ERR_INVALID_CONFIG, "dimension must be greater than 0");
    if (p.codebook_size > 256)
        throw Error(VGPU_ERR_INVALID_CONFIG,
                    "codebook_size must be at most 256 because PQ codes are stored as u8");
    VGPU_HIP(hipGetDevice(&device));
    VGPU_HIP(hipStreamCreateWithFlags(&stream, hipStreamNonBlocking));
}

IvfpqIndex::~IvfpqIndex() {
    ws_pool.clear();
    if (stream) (void)hipStreamSynchronize(stream);
    if (stream) (void)hipStreamDestroy(stream);
}

void IvfpqIndex::add(const uint32_t* ids, const float* x, size_t count) {
    if (built) throw Error(VGPU_ERR_ALREADY_BUILT, "IVF-PQ index: cannot add vectors after build");
    for (size_t i = 0; i < count * d; i++)
        if (!std::isfinite(x[i])) throw Error(VGPU_ERR_INVALID_PARAMETER, "vector contains a non-finite value");
    size_t base = vectors.size();
    vectors.resize(base + count * d);
    for (size_t i = 0; i < count; i++) normalize_row(x + i * d, d, vectors.data() + base + i * d);
    doc_ids.insert(doc_ids.end(), ids, ids + count);
}

// argmin over centroids of 1 - dot(x, c), lowest index on ties: the coarse
// kernels with nprobe = 1 on the rows as given (they are already normalised).
// The fused kernel needs no score matrix; the GEMM fallback (d > 128) is
// chunked to bound the score matrix at 1 GiB.
void IvfpqIndex::assign_cosine(const float* d_x, const float* d_norms, size_t nx,
                               const float* d_cent, size_t k, float cmax, uint32_t* d_assign,
                               hipStream_t s) {
    if (coarse_fused_supported((int)d, 1)) {
        const size_t chunk = std::min<size_t>(nx, (size_t)1 << 18);
        b_cb16.reserve(coarse_bf16_pack_chunks((int)k, (int)d));
        b_cflag_list.reserve(chunk);
        b_cflag_count.reserve(1);
        b_overflow.reserve(1);
        VGPU_HIP(hipMemsetAsync(b_overflow.p, 0, sizeof(unsigned int), s));
        launch_coarse_bf16_pack(d_cent, (int)k, (int)d, b_cb16.p, s);
        for (size_t q0 = 0; q0 < nx; q0 += chunk) {
            const size_t nc = std::min(chunk, nx - q0);
            VGPU_HIP(hipMemsetAsync(b_cflag_count.p, 0, sizeof(uint32_t), s));
            launch_coarse_fused(d_x + q0 * d, (int)nc, (int)d, b_cb16.p, (int)k, cmax, 1, 0, 0, nullptr,
                                nullptr, d_cent, d_assign + q0, b_cflag_list.p, b_cflag_count.p, s);
            launch_coarse_exact_flagged(d_x + q0 * d, d_norms + q0, d_cent, (int)nc, (int)k, (int)d, 1,
                                        cmax, d_assign + q0, b_overflow.p, b_cflag_list.p,
                                        b_cflag_count.p, s);
        }
        VGPU_HIP(hipGetLastError());
        return;
    }
    size_t chunk = std::max<size_t>(1, std::min<size_t>(nx, ((size_t)1 << 28) / std::max<size_t>(k, 1)));
    chunk = std::min<size_t>(chunk, (size_t)1 << 20);  // grid.y of the GEMM stays < 65536
    b_dots.reserve(chunk * k);
    b_cflag_list.reserve(chunk);
    b_cflag_count.reserve(1);
    b_overflow.reserve(1);
    VGPU_HIP(hipMemsetAsync(b_overflow.p, 0, sizeof(unsigned int), s));
    for (size_t q0 = 0; q0 < nx; q0 += chunk) {
        size_t nc = std::min(chunk, nx - q0);
        launch_coarse_dots(d_x + q0 * d, d_cent, b_dots.p, (int)nc, (int)k, (int)d, s);
        VGPU_HIP(hipMemsetAsync(b_cflag_count.p, 0, sizeof(uint32_t), s));
        launch_coarse_select(b_dots.p, d_x + q0 * d, d_norms + q0, d_cent, (int)nc, (int)k, (int)d, 1,
                             cmax, d_assign + q0, b_overflow.p, b_cflag_list.p, b_cflag_count.p, s);
    }
    VGPU_HIP(hipGetLastError());
}

// Lloyd k-means with cosine assignment (the role of clump's CosineDistance
// k-means, src/partitioning/kmeans.rs:64-107): k_eff = min(k, n) seeded
// distinct starting points; assign on the GPU; stop when no assignment
// changes; otherwise each non-empty centroid becomes the float64 mean of its
// members (index order), re-normalised.  Both steps run on the GPU for
// d <= 256 (the update kernel's row width); the host keeps the assignment
// test and the centroid norm bound.
void IvfpqIndex::kmeans_cosine(const std::vector<float>& x, size_t nt, size_t k, uint64_t seed,
                               size_t max_iter, std::vector<float>& cent) {
    const size_t ke = std::min(k, nt);
    std::vector<uint32_t> init;
    draw_distinct(nt, ke, seed, init);
    cent.assign(ke * d, 0.0f);
    for (size_t c = 0; c < ke; c++) std::memcpy(&cent[c * d], &x[(size_t)init[c] * d], d * sizeof(float));
    std::vector<float> norms(nt);
    for (size_t i = 0; i < nt; i++) norms[i] = row_norm_bound(&x[i * d], d);
    DevBuf<float> dx, dn, dc;
    DevBuf<uint32_t> da;
    dx.upload(x.data(), nt * d, stream);
    dn.upload(norms.data(), nt, stream);
    da.reserve(nt);
    std::vector<uint32_t> assign(nt), prev(nt);
    const bool gpu_update = d <= 256;
    DevBuf<uint32_t> dks;  // member lists of the update
    if (gpu_update) dks.reserve(kmeans_update_scratch_words((int)nt, 1, (int)ke));
    dc.upload(cent.data(), ke * d, stream);
    for (size_t it = 0; it < max_iter; it++) {
        float cmax = 0.0f;
        for (size_t c = 0; c < ke; c++) cmax = std::max(cmax, row_norm_bound(&cent[c * d], d));
        if (!gpu_update) dc.upload(cent.data(), ke * d, stream);
        assign_cosine(dx.p, dn.p, nt, dc.p, ke, cmax, da.p, stream);
        VGPU_HIP(hipMemcpyAsync(assign.data(), da.p, nt * sizeof(uint32_t), hipMemcpyDeviceToHost, stream));
        VGPU_HIP(hipStreamSynchronize(stream));
        check_labels(assign.data(), nt, 1, ke, "k-means assignment");
        if (it > 0 && assign == prev) break;
        if (gpu_update) {
            VGPU_HIP(launch_kmeans_update(dx.p, (int)nt, (int)d, (int)d, 1, da.p, false, (int)ke, nullptr, true,
                                          dc.p, dks.p, dks.n, stream));
            VGPU_HIP(hipMemcpyAsync(cent.data(), dc.p, ke * d * sizeof(float), hipMemcpyDeviceToHost, stream));
            VGPU_HIP(hipStreamSynchronize(stream));
            prev.swap(assign);
            continue;
        }
        centroid_update(x.data(), nt, d, assign.data(), ke, cent.data());
        prev.swap(assign);
    }
}

// One squared-L2 k-means per subspace (pq.rs:75-124, seed + m), all M run
// together: one GPU encode pass assigns every subspace; a subspace whose
// assignment stopped changing is frozen, exactly as if it had been run alone.
// The codeword means run on the GPU (float64, member order) for ds <= 256.
void IvfpqIndex::train_pq(const std::vector<float>& res, size_t nt, size_t Kc, uint64_t seed,
                          size_t max_iter) {
    const size_t Ke = std::min(Kc, nt);
    K = Ke;
    codebooks.assign(M * Ke * ds, 0.0f);
    std::vector<uint32_t> init;
    for (size_t m = 0; m < M; m++) {
        draw_distinct(nt, Ke, seed + m, init);
        for (size_t c = 0; c < Ke; c++)
            std::memcpy(&codebooks[(m * Ke + c) * ds], &res[(size_t)init[c] * d + m * ds], ds * sizeof(float));
    }
    DevBuf<float> dres, dcb;
    DevBuf<uint8_t> dcodes, dactive;
    dres.upload(res.data(), nt * d, stream);
    dcodes.reserve(nt * M);
    std::vector<uint8_t> cur(nt * M), prev(nt * M), active(M);
    std::vector<char> frozen(M, 0);
    // the update's member lists hold 32-bit row indices of every subspace
    const bool gpu_update = ds <= 256 && (uint64_t)nt * M < ((uint64_t)1 << 32);
    DevBuf<uint32_t> dks;  // member lists of the update
    if (gpu_update) dks.reserve(kmeans_update_scratch_words((int)nt, (int)M, (int)Ke));
    dcb.upload(codebooks.data(), codebooks.size(), stream);
    for (size_t it = 0; it < max_iter; it++) {
        if (!gpu_update) dcb.upload(codebooks.data(), codebooks.size(), stream);
        launch_encode(dres.p, (int)nt, (int)d, nullptr, nullptr, dcb.p, (int)M, (int)Ke, (int)ds,
                      dcodes.p, stream);
        VGPU_HIP(hipGetLastError());
        VGPU_HIP(hipMemcpyAsync(cur.data(), dcodes.p, nt * M, hipMemcpyDeviceToHost, stream));
        VGPU_HIP(hipStreamSynchronize(stream));
        check_labels(cur.data(), nt * M, 1, Ke, "PQ codes");
        bool any = false;
        for (size_t m = 0; m < M; m++) {
            active[m] = 0;
            if (frozen[m]) continue;
            if (it > 0) {
                bool same = true;
                for (size_t i = 0; i < nt && same; i++) same = cur[i * M + m] == prev[i * M + m];
                if (same) {
                    frozen[m] = 1;
                    continue;
                }
            }
            any = true;
            active[m] = 1;
            if (gpu_update) continue;
            host_mean_update(res.data(), nt, d, m * ds, ds, cur.data() + m, M, Ke, false,
                             &codebooks[m * Ke * ds]);
        }
        if (!any) break;
        if (gpu_update) {
            dactive.upload(active.data(), M, stream);
            VGPU_HIP(launch_kmeans_update(dres.p, (int)nt, (int)d, (int)ds, (int)M, dcodes.p, true, (int)Ke,
                                          dactive.p, false, dcb.p, dks.p, dks.n, stream));
        }
        prev.swap(cur);
    }
    if (gpu_update) {
        VGPU_HIP(hipMemcpyAsync(codebooks.data(), dcb.p, codebooks.size() * sizeof(float),
                                hipMemcpyDeviceToHost, stream));
        VGPU_HIP(hipStreamSynchronize(stream));
    }
}

void IvfpqIndex::build(size_t sample, size_t max_iter) {
    if (built) return;  // search.rs:550-552
    const size_t n = this->n();
    if (n == 0) throw Error(VGPU_ERR_EMPTY_INDEX, "index is empty");
    if (n < params.codebook_size)
        throw Error(VGPU_ERR_INVALID_PARAMETER,
                    "IVF-PQ requires at least codebook_size training vectors (got " +
                        std::to_string(n) + " vectors, codebook_size = " +
                        std::to_string(params.codebook_size) + ")");
    if (max_iter == 0) throw Error(VGPU_ERR_INVALID_CONFIG, "kmeans_max_iter must be greater than 0");
    std::vector<uint32_t> tidx;
    sample_indices(n, sample, params.seed, tidx);
    const size_t nt = tidx.size();
    size_t min_train = std::max(std::min(params.num_clusters, n), params.codebook_size);
    if (nt < min_train)
        throw Error(VGPU_ERR_INVALID_PARAMETER, "IVF-PQ training sample is too small (got " +
                                                    std::to_string(nt) + ", need at least " +
                                                    std::to_string(min_train) + ")");
    if (params.num_clusters == 0)
        throw Error(VGPU_ERR_INVALID_CONFIG, "dimension and k must both be greater than 0");
    if (params.num_codebooks == 0 || params.codebook_size == 0)
        throw Error(VGPU_ERR_INVALID_CONFIG,
                    "dimension, num_codebooks, codebook_size must all be greater than 0");
    if (d % params.num_codebooks)
        throw Error(VGPU_ERR_INVALID_CONFIG, "dimension must be divisible by num_codebooks");
    if (params.use_opq && d > 2048)
        throw Error(VGPU_ERR_UNSUPPORTED, "OPQ rotation is limited to dimension <= 2048");
    if (n >= 0xffffffffull) throw Error(VGPU_ERR_INVALID_PARAMETER, "more than 2^32-1 vectors");
    M = params.num_codebooks;
    ds = d / M;

    std::vector<float> train(nt * d);
    for (size_t i = 0; i < nt; i++) std::memcpy(&train[i * d], &vectors[(size_t)tidx[i] * d], d * sizeof(float));
    kmeans_cosine(train, nt, params.num_clusters, params.seed, max_iter, centroids);
    L = centroids.size() / d;

    // List assignment of every vector (search.rs:621).
    float cmax = 0.0f;
    for (size_t c = 0; c < L; c++) cmax = std::max(cmax, row_norm_bound(&centroids[c * d], d));
    std::vector<float> norms(n);
    for (size_t i = 0; i < n; i++) norms[i] = row_norm_bound(&vectors[i * d], d);
    d_vectors.upload(vectors.data(), n * d, stream);
    d_centroids.upload(centroids.data(), L * d, stream);
    DevBuf<float> dn;
    DevBuf<uint32_t> dassign;
    dn.upload(norms.data(), n, stream);
    dassign.reserve(n);
    assign_cosine(d_vectors.p, dn.p, n, d_centroids.p, L, cmax, dassign.p, stream);
    std::vector<uint32_t> assign(n);
    VGPU_HIP(hipMemcpyAsync(assign.data(), dassign.p, n * sizeof(uint32_t), hipMemcpyDeviceToHost, stream));
    VGPU_HIP(hipStreamSynchronize(stream));

    // Lists: insertion order inside a list (search.rs:624-657); the labels are
    // range-checked there, before the residuals below index the centroids.
    build_lists(assign.data(), n, L, offsets, list_ids);

    // Residual PQ training on the sample (search.rs:722-772).
    std::vector<float> res(nt * d);
    for (size_t i = 0; i < nt; i++) {
        const uint32_t v = tidx[i];
        const float* c = &centroids[(size_t)assign[v] * d];
        for (size_t j = 0; j < d; j++) res[i * d + j] = vectors[(size_t)v * d + j] - c[j];
    }
    rotation.clear();
    if (params.use_opq)
        train_opq(res, nt, params.seed);  // opq.fit(training, count, 10), search.rs:732-749
    else
        train_pq(res, nt, params.codebook_size, params.seed, max_iter);

    // Encode every residual (search.rs:776-781); OPQ rotates it first
    // (opq.rs:112-115), a chunk of rows at a time.
    d_codebooks.upload(codebooks.data(), codebooks.size(), stream);
    DevBuf<uint8_t> dcodes;
    dcodes.reserve(n * M);
    if (!rotation.empty()) {
        d_rotation.upload(rotation.data(), d * d, stream);
        const size_t chunk = std::max<size_t>(1, std::min<size_t>(n, ((size_t)1 << 28) / d));
        DevBuf<float> drx;
        drx.reserve(chunk * d);
        for (size_t r0 = 0; r0 < n; r0 += chunk) {
            const size_t nc = std::min(chunk, n - r0);
            launch_rotate_rows(d_rotation.p, d_vectors.p + r0 * d, 1, d_centroids.p, dassign.p + r0, (int)L,
                               nc, (int)d, drx.p, stream);
            launch_encode(drx.p, (int)nc, (int)d, nullptr, nullptr, d_codebooks.p, (int)M, (int)K, (int)ds,
                          dcodes.p + r0 * M, stream);
        }
        VGPU_HIP(hipGetLastError());
        VGPU_HIP(hipStreamSynchronize(stream));
    } else {
        launch_encode(d_vectors.p, (int)n, (int)d, d_centroids.p, dassign.p, d_codebooks.p, (int)M,
                      (int)K, (int)ds, dcodes.p, stream);
    }
    VGPU_HIP(hipGetLastError());
    codes.resize(n * M);
    VGPU_HIP(hipMemcpyAsync(codes.data(), dcodes.p, n * M, hipMemcpyDeviceToHost, stream));
    VGPU_HIP(hipStreamSynchronize(stream));
    check_labels(codes.data(), n * M, 1, K, "PQ codes");
    has_vectors = true;
    upload_index();
    built = true;
}

void IvfpqIndex::load(const float* cent, size_t Lc, const float* cb, size_t Kc,
                      const uint64_t* off, const uint32_t* lids, const uint8_t* cds,
                      const uint32_t* dids, const float* vecs, size_t nv) {
    if (params.num_codebooks == 0 || d % params.num_codebooks)
        throw Error(VGPU_ERR_INVALID_CONFIG, "dimension must be divisible by num_codebooks");
    if (Lc == 0 || Kc == 0 || Kc > 256)
        throw Error(VGPU_ERR_INVALID_CONFIG, "need num_centroids > 0 and 1 <= codebook_size <= 256");
    if (nv >= 0xffffffffull) throw Error(VGPU_ERR_INVALID_PARAMETER, "more than 2^32-1 vectors");
    M = params.num_codebooks;
    ds = d / M;
    L = Lc;
    K = Kc;
    if (off[0] != 0 || off[L] != nv)
        throw Error(VGPU_ERR_INVALID_PARAMETER, "list_offsets must start at 0 and end at num_vectors");
    for (size_t l = 0; l < L; l++)
        if (off[l + 1] < off[l]) throw Error(VGPU_ERR_INVALID_PARAMETER, "list_offsets must be non-decreasing");
    std::vector<char> seen(nv, 0);
    for (size_t i = 0; i < nv; i++) {
        if (lids[i] >= nv || seen[lids[i]])
            throw Error(VGPU_ERR_INVALID_PARAMETER, "list_ids must be a permutation of 0..num_vectors");
        seen[lids[i]] = 1;
    }
    for (size_t i = 0; i < nv * M; i++)
        if (cds[i] >= K) throw Error(VGPU_ERR_INVALID_PARAMETER, "code outside the codebook");
    centroids.assign(cent, cent + L * d);
    codebooks.assign(cb, cb + M * K * ds);
    offsets.assign(off, off + L + 1);
    list_ids.assign(lids, lids + nv);
    codes.assign(cds, cds + nv * M);
    doc_ids.resize(nv);
    for (size_t i = 0; i < nv; i++) doc_ids[i] = dids ? dids[i] : (uint32_t)i;
    if (vecs) {
        vectors.assign(vecs, vecs + nv * d);
        has_vectors = true;
    } else {
        vectors.clear();
        has_vectors = false;
    }
    if (has_vectors) d_vectors.upload(vectors.data(), nv * d, stream);
    d_centroids.upload(centroids.data(), L * d, stream);
    d_codebooks.upload(codebooks.data(), codebooks.size(), stream);
    upload_index();
    built = true;
}

// HBM layout of the search path (the list-major caches of
// build_scan_caches, search.rs:816-848, plus the FAST term).
void IvfpqIndex::upload_index() {
    const size_t n = this->n();
    snapshot_list_masks();
    std::vector<uint32_t> off32(L + 1);
    for (size_t l = 0; l <= L; l++) off32[l] = (uint32_t)offsets[l];
    std::vector<uint8_t> lm(n * M);
    for (size_t p = 0; p < n; p++) std::memcpy(&lm[p * M], &codes[(size_t)list_ids[p] * M], M);
    d_offsets.upload(off32.data(), L + 1, stream);
    d_list_ids.upload(list_ids.data(), n, stream);
    d_doc_ids.upload(doc_ids.data(), n, stream);
    d_codes.upload(lm.data(), n * M, stream);
    if (!has_vectors) d_vectors.release();

    double cm = 0.0;
    for (size_t c = 0; c < L; c++) cm = std::max(cm, (double)row_norm_bound(&centroids[c * d], d));
    double rr = 0.0;
    for (size_t m = 0; m < M; m++) {
        double best = 0.0;
        for (size_t k = 0; k < K; k++) {
            double s = 0.0;
            for (size_t j = 0; j < ds; j++) {
                double v = codebooks[(m * K + k) * ds + j];
                s += v * v;
            }
            best = std::max(best, s);
        }
        rr += best;
    }
    dix = DevIndex{};
    dix.d = (int)d;
    dix.L = (int)L;
    dix.M = (int)M;
    dix.K = (int)K;
    dix.ds = (int)ds;
    dix.n = (uint32_t)n;
    dix.centroids = d_centroids.p;
    d_cb16.reserve(coarse_bf16_pack_chunks((int)L, (int)d));
    launch_coarse_bf16_pack(d_centroids.p, (int)L, (int)d, d_cb16.p, stream);
    dix.cb16 = d_cb16.p;
    dix.codebooks = d_codebooks.p;
    dix.offsets = d_offsets.p;
    dix.list_ids = d_list_ids.p;
    dix.codes = d_codes.p;
    dix.doc_ids = d_doc_ids.p;
    dix.vectors = has_vectors ? d_vectors.p : nullptr;
    dix.cmax = (float)(cm * 1.0001);
    dix.rmax = (float)(std::sqrt(rr) * 1.0001 + 1e-30);
    if (!rotation.empty()) d_rotation.upload(rotation.data(), d * d, stream);
    else d_rotation.release();
    if (K == 16) {
        std::vector<uint32_t> poff(L + 1, 0);
        for (size_t l = 0; l < L; l++) {
            uint64_t len = offsets[l + 1] - offsets[l];
            poff[l + 1] = poff[l] + (len >= 16 ? (uint32_t)((len + 31) / 32) : 0u);
        }
        // the FastScan kernel addresses the packed blocks with 32-bit byte offsets
        if ((uint64_t)poff[L] * 16 * M >= ((uint64_t)1 << 32))
            throw Error(VGPU_ERR_UNSUPPORTED, "4-bit packed codes of " + std::to_string((uint64_t)poff[L] * 16 * M) +
                                                  " bytes: FastScan addresses at most 4 GiB");
        d_pack_off.upload(poff.data(), L + 1, stream);
        d_packed.reserve((size_t)poff[L] * 16 * M + 16);
        dix.pack_off = d_pack_off.p;
        dix.packed = d_packed.p;
        launch_pack4(dix, d_packed.p, stream);
        d_bias.release();
    } else if (!rotation.empty()) {  // OPQ scans in EXACT mode: no FAST arrays
        d_bias.release();
        d_tblocks.release();
        d_tblk_off.release();
        dix.bias = nullptr;
        dix.tcodes = nullptr;
        dix.tbias = nullptr;
        dix.tblk_off = nullptr;
    } else {
        d_bias.reserve(n);
        dix.bias = d_bias.p;
        launch_bias(dix, d_bias.p, stream);
        std::vector<uint32_t> toff(L + 1, 0);
        for (size_t l = 0; l < L; l++)
            toff[l + 1] = toff[l] + (uint32_t)((offsets[l + 1] - offsets[l] + 15) / 16);
        const size_t nblk = (size_t)toff[L] + 1;  // + one block of slack
        // lane records are indexed by 32-bit structured-buffer indices
        if (scan8_fast_blocks_supported((int)M, (int)K, (int)ds) && nblk * 16 < ((size_t)1 << 31)) {
            d_tblk_off.upload(toff.data(), L + 1, stream);
            d_tblocks.reserve(nblk * TBLK_BYTES(M));  // codes, then the b(x) floats
            dix.tblk_off = d_tblk_off.p;
            dix.tcodes = d_tblocks.p;
            dix.tbias = reinterpret_cast<float*>(d_tblocks.p + nblk * 16 * M);
            dix.tblk_count = (uint32_t)nblk;
            launch_tblocks(dix, d_tblocks.p, const_cast<float*>(dix.tbias), stream);
        } else {
            d_tblocks.release();
            d_tblk_off.release();
        }
    }
    VGPU_HIP(hipGetLastError());
    VGPU_HIP(hipStreamSynchronize(stream));
}

static int fast_keep(size_t kout) {
    int kk = 1;
    while ((size_t)kk < kout + 16) kk <<= 1;
    return std::max(kk, 32);
}

SearchWs::SearchWs() {
    // non-blocking: no implicit wait on the null stream (default priority)
    VGPU_HIP(hipStreamCreateWithFlags(&stream, hipStreamNonBlocking));

    for (auto& e : ev) VGPU_HIP(hipEventCreate(&e));
    VGPU_HIP(hipHostMalloc((void**)&h_scal, kScalWords * sizeof(unsigned long long)));
}

SearchWs::~SearchWs() {
    if (stream) (void)hipStreamSynchronize(stream);

    if (h_scal) (void)hipHostFree(h_scal);
    for (auto& e : ev)
        if (e) (void)hipEventDestroy(e);
    for (auto& e : sev)
        if (e) (void)hipEventDestroy(e);
    if (stream) (void)hipStreamDestroy(stream);
}

std::unique_ptr<SearchWs> IvfpqIndex::take_ws() {
    {
        std::lock_guard<std::mutex> lk(pool_mu);
        if (!ws_pool.empty()) {
            auto ws = std::move(ws_pool.back());
            ws_pool.pop_back();
            return ws;
        }
    }
    return std::make_unique<SearchWs>();
}

void IvfpqIndex::give_ws(std::unique_ptr<SearchWs> ws) {
    std::lock_guard<std::mutex> lk(pool_mu);
    ws_pool.push_back(std::move(ws));
}

namespace {
// Returns a borrowed workspace to the pool when the call ends, thrown or
// not, after the work queued on it (on the call's stream) has finished.
struct WsLease {
    IvfpqIndex& ix;
    std::unique_ptr<SearchWs> ws;
    hipStream_t used = nullptr;  // the stream the call queued its work on
    WsLease(IvfpqIndex& i, std::unique_ptr<SearchWs> w) : ix(i), ws(std::move(w)) {}
    ~WsLease() {
        if (ws) {
            (void)hipStreamSynchronize(used ? used : ws->stream);
            ix.give_ws(std::move(ws));
        }
    }
    SearchWs* operator->() { return ws.get(); }
};
}  // namespace

vgpu_search_stats IvfpqIndex::last_stats() {
    std::lock_guard<std::mutex> lk(stats_mu);
    return stats;
}

SearchPlan IvfpqIndex::plan_search(size_t nq, size_t k, size_t nprobe, size_t pool) const {
    SearchPlan pl;
    if (pool && !has_vectors)
        throw Error(VGPU_ERR_UNSUPPORTED, "search_reranked after compact(): raw vectors were dropped");
    pl.P = std::min(nprobe ? nprobe : params.nprobe, L);  // search.rs:1610
    pl.k = k;
    pl.pool = pool;
    pl.kout = pool ? std::max(pool, k) : k;  // search.rs:1144
    if (pool && pl.kout > RERANK_MAX)
        throw Error(VGPU_ERR_UNSUPPORTED, "rerank_pool above " + std::to_string(RERANK_MAX) + " is not supported");
    pl.wide = pl.P > 1024 || pl.kout > 2048;
    if (pl.P > SEL_WIDE_MAX)  // min(nprobe, nlist) lists sorted in LDS
        throw Error(VGPU_ERR_UNSUPPORTED, "probing more than " + std::to_string(SEL_WIDE_MAX) +
                                              " lists is not supported");
    if (pl.P) {
        ScanArgs probe_shape;
        probe_shape.P = (int)pl.P;
        probe_shape.kout = (int)pl.kout;
        size_t lds;
        if (K == 16) {
            probe_shape.kk = (int)pl.kout;
            lds = fastscan_lds_bytes(dix, probe_shape);
        } else if (pl.wide) {  // EXACT only
            probe_shape.kk = (int)pl.kout;
            lds = scan8_lds_bytes(dix, probe_shape);
        } else {
            probe_shape.kk = fast_keep(pl.kout);
            lds = scan8_fast_lds_bytes(dix, probe_shape);
            probe_shape.kk = (int)pl.kout;
            lds = std::max(lds, scan8_lds_bytes(dix, probe_shape));
        }
        if (lds > 160 * 1024)
            throw Error(VGPU_ERR_UNSUPPORTED, "k of " + std::to_string(pl.kout) + " needs a scan working set of " +
                                                  std::to_string(lds) +
                                                  " bytes, above the 160 KiB of LDS per workgroup");
    }
    pl.opq = !rotation.empty();
    pl.fused = coarse_fused_supported((int)d, (int)pl.P);
    pl.t2 = pl.P && K != 16 && mode == VGPU_MODE_FAST && !pl.opq && !pl.wide && scan8_fast_uses_tables(dix);
    size_t chunk = std::max<size_t>(1, std::min<size_t>(nq, ((size_t)1 << 28) / std::max<size_t>(L, 1)));
    chunk = std::min<size_t>(chunk, 65536);
    if (pl.t2)  // tables of a chunk within 256 MiB
        chunk = std::max<size_t>(1, std::min<size_t>(chunk, ((size_t)1 << 26) / ((size_t)M * K)));
    if (pl.opq && pl.P)
        chunk = std::max<size_t>(1, std::min<size_t>(chunk, ((size_t)1 << 28) / (pl.P * d)));
    pl.chunk = chunk;
    return pl;
}

size_t IvfpqIndex::ws_layout(const SearchPlan& pl, uint8_t* base, WsPtrs* out) const {
    size_t off = 0;
    auto carve = [&](auto*& p, size_t count) {
        using T = std::remove_reference_t<decltype(*p)>;
        off = (off + 255) & ~(size_t)255;
        if (base) p = reinterpret_cast<T*>(base + off);
        off += std::max<size_t>(count, 1) * sizeof(T);
    };
    WsPtrs w;
    const size_t c = pl.chunk;
    carve(w.scal, kScalWords);
    carve(w.qn, c * d);
    carve(w.qnorm, c);
    carve(w.qbad, c);
    if (pl.fused) {
        carve(w.fdots, (size_t)COARSE_FLAG_PAR * L);
    } else if (pl.P) {
        carve(w.dots, c * L);
    }
    carve(w.cflag_list, c);
    carve(w.probe, c * std::max<size_t>(pl.P, 1));
    carve(w.vidx, c * pl.kout);
    carve(w.dist, c * pl.kout);
    if (pl.pool) {
        carve(w.vidx2, c * pl.k);
        carve(w.dist2, c * pl.k);
    }
    carve(w.qstat, c * QSTAT_WORDS);
    carve(w.flag_list, c);
    if (pl.opq) carve(w.rres, c * pl.P * d);
    if (pl.t2) carve(w.t2, c * M * K);
    if (out) *out = w;
    return (off + 255) & ~(size_t)255;
}

// Normalise (search.rs:55-62) and probe (search.rs:1602-1617) nq <= chunk
// queries.  The fused path normalises in its prologue; P == 0 only normalises.
void IvfpqIndex::coarse_probe(const float* d_q, size_t nq, size_t P, const SearchPlan& pl,
                              const WsPtrs& w, hipStream_t s, hipEvent_t mid, bool ordered) {
    unsigned int* overflow = reinterpret_cast<unsigned int*>(w.scal + kOverflowWord);
    uint32_t* cflag_count = reinterpret_cast<uint32_t*>(w.scal + kCFlagWord);
    unsigned int* nbad = reinterpret_cast<unsigned int*>(w.scal + kBadWord);
    if (P == 0) {
        launch_normalize(d_q, w.qn, w.qnorm, (int)nq, (int)d, s, w.qbad, nbad);
        return;
    }
    if (pl.fused) {
        launch_coarse_fused(d_q, (int)nq, (int)d, dix.cb16, (int)L, dix.cmax, (int)P, 1, ordered ? 1 : 0, w.qn, w.qnorm,
                            d_centroids.p, w.probe, w.cflag_list, cflag_count, s, w.qbad, nbad);
        if (mid) VGPU_HIP(hipEventRecord(mid, s));
        launch_coarse_exact_flagged(w.qn, w.qnorm, d_centroids.p, (int)nq, (int)L, (int)d, (int)P, dix.cmax,
                                    w.probe, overflow, w.cflag_list, cflag_count, s, w.fdots,
                                    reinterpret_cast<uint32_t*>(w.scal + kFDoneWord));
    } else if (P > 1024) {  // every list's exact score, then the P smallest
        launch_normalize(d_q, w.qn, w.qnorm, (int)nq, (int)d, s, w.qbad, nbad);
        if (mid) VGPU_HIP(hipEventRecord(mid, s));
        launch_coarse_select_wide(w.dots, w.qn, d_centroids.p, (int)nq, (int)L, (int)d, (int)P, w.probe, s);
    } else {
        launch_normalize(d_q, w.qn, w.qnorm, (int)nq, (int)d, s, w.qbad, nbad);
        launch_coarse_dots(w.qn, d_centroids.p, w.dots, (int)nq, (int)L, (int)d, s);
        if (mid) VGPU_HIP(hipEventRecord(mid, s));
        launch_coarse_select(w.dots, w.qn, w.qnorm, d_centroids.p, (int)nq, (int)L, (int)d, (int)P, dix.cmax,
                             w.probe, overflow, w.cflag_list, cflag_count, s);
    }
}

// A query holding a NaN or an infinity is searched as the zero vector and its
// row padded; the call then reports it, like the host entry points.
static void check_nonfinite(unsigned long long word) {
    const unsigned int n = (unsigned int)(word & 0xffffffffu);
    if (n)
        throw Error(VGPU_ERR_INVALID_PARAMETER, "query contains a non-finite value (" + std::to_string(n) +
                                                    " queries; their rows are padding)");
}

// End of an allocation-free call.  Under stream capture nothing may wait on
// the stream: the call returns with its work recorded, completion is the
// caller's, and non-finite queries show only as padding rows.  Otherwise wait,
// then read the non-finite count back with a synchronous 4-byte copy (no
// allocation).
static void complete_noalloc(const WsPtrs& w, hipStream_t s) {
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    VGPU_HIP(hipStreamIsCapturing(s, &cs));
    if (cs != hipStreamCaptureStatusNone) return;
    VGPU_HIP(hipStreamSynchronize(s));
    unsigned int nbad = 0;
    VGPU_HIP(hipMemcpy(&nbad, w.scal + kBadWord, sizeof(nbad), hipMemcpyDeviceToHost));
    check_nonfinite(nbad);
}

void IvfpqIndex::run_search(const float* d_q, size_t nq, const SearchPlan& pl, const WsPtrs& w,
                            int64_t* d_ids, float* d_dists, hipStream_t s, SearchWs* ws,
                            vgpu_search_stats* st, const uint32_t* d_given) {
    const size_t P = pl.P, k = pl.k, kout = pl.kout, chunk = pl.chunk;
    unsigned long long* counters = w.scal;
    uint32_t* flag_count = reinterpret_cast<uint32_t*>(w.scal + kFlagWord);
    uint32_t* cflag_count = reinterpret_cast<uint32_t*>(w.scal + kCFlagWord);
    launch_zero_words(w.scal, kScalWords, s);
    if (P == 0) {  // no probed list: every row is padding (the queries are still checked)
        for (size_t q0 = 0; q0 < nq; q0 += chunk)
            launch_normalize(d_q + q0 * d, w.qn, w.qnorm, (int)std::min(chunk, nq - q0), (int)d, s,
                             nullptr, reinterpret_cast<unsigned int*>(w.scal + kBadWord));
        launch_finalize(nullptr, nullptr, nullptr, (int)nq, 0, (int)k, d_ids, d_dists, s);
        VGPU_HIP(hipGetLastError());
        if (!ws) {
            complete_noalloc(w, s);
            return;
        }
        VGPU_HIP(hipMemcpyAsync(ws->h_scal, w.scal, kScalWords * sizeof(unsigned long long),
                                hipMemcpyDeviceToHost, s));
        VGPU_HIP(hipStreamSynchronize(s));
        check_nonfinite(ws->h_scal[kBadWord]);
        return;
    }
    float t[7] = {0, 0, 0, 0, 0, 0, 0}, t_table = 0;
    const int prof = ws ? profiling : 0;
    const bool allp = prof == 1, scanp = prof == 2;
    if (scanp) {
        const size_t need_ev = 4 * ((nq + chunk - 1) / chunk);
        while (ws->sev.size() < need_ev) {
            hipEvent_t e;
            VGPU_HIP(hipEventCreate(&e));
            ws->sev.push_back(e);
        }
    }
    hipEvent_t* ev = ws ? ws->ev : nullptr;
    size_t ci = 0;  // chunk index
    for (size_t q0 = 0; q0 < nq; q0 += chunk, ci++) {
        const size_t nc = std::min(chunk, nq - q0);
        if (allp) VGPU_HIP(hipEventRecord(ev[0], s));
        // normalise + bf16x3 MFMA pass or score GEMM (ms_coarse), exact top-P
        // of the candidates and the rare exact fallback (ms_select)
        if (allp) VGPU_HIP(hipEventRecord(ev[1], s));
        const uint32_t* probe = w.probe;
        if (d_given) {
            launch_normalize(d_q + q0 * d, w.qn, w.qnorm, (int)nc, (int)d, s, w.qbad,
                             reinterpret_cast<unsigned int*>(w.scal + kBadWord));
            if (allp) VGPU_HIP(hipEventRecord(ev[2], s));
            probe = d_given + q0 * P;
        } else {
            coarse_probe(d_q + q0 * d, nc, P, pl, w, s, allp ? ev[2] : nullptr);
        }
        // OPQ: the rotated residual of every (query, probe) slot (opq.rs:120-123),
        // timed with the selection
        if (pl.opq) rotate_slots(w.qn, nc, P, probe, w.rres, s);
        if (allp) VGPU_HIP(hipEventRecord(ev[3], s));
        // scan-only timing: the FAST kernel's dispatch records the two events
        // itself; the other scan kernels are bracketed by marker events
        const bool scan_fast = K != 16 && mode == VGPU_MODE_FAST && !pl.opq && !pl.wide;
        if (scanp && !scan_fast) VGPU_HIP(hipEventRecord(ws->sev[4 * ci], s));
        ScanArgs a;
        a.qn = w.qn;
        a.qnorm = w.qnorm;
        a.probe = probe;
        a.nq = (int)nc;
        a.P = (int)P;
        a.kout = (int)kout;
        a.qstat = w.qstat;
        a.flag_list = w.flag_list;
        a.flag_count = flag_count;
        a.out_vidx = w.vidx;
        a.out_dist = w.dist;
        if (!pl.pool) {  // no rerank: the scan kernels write the final rows
            a.out_ids = d_ids + q0 * k;
            a.out_dists = d_dists + q0 * k;
            a.doc_ids = d_doc_ids.p;
        }
        a.rres = pl.opq ? w.rres : nullptr;
        if (K == 16) {
            a.kk = (int)kout;
            launch_fastscan(dix, a, s);
            if (allp) VGPU_HIP(hipEventRecord(ev[4], s));
            if (scanp) VGPU_HIP(hipEventRecord(ws->sev[4 * ci + 1], s));
        } else if (scan_fast) {
            a.kk = fast_keep(kout);
            a.exact = 0;
            if (pl.t2) {  // the per-query tables (ms_table)
                launch_t2_tables(dix, w.qn, (int)nc, w.t2, s, scanp ? ws->sev[4 * ci + 2] : nullptr,
                                 scanp ? ws->sev[4 * ci + 3] : nullptr);
                if (allp) VGPU_HIP(hipEventRecord(ev[8], s));
                a.t2 = w.t2;
            }
            launch_scan8_fast(dix, a, s, scanp ? ws->sev[4 * ci] : nullptr, scanp ? ws->sev[4 * ci + 1] : nullptr);
            if (allp) VGPU_HIP(hipEventRecord(ev[4], s));
            a.kk = (int)kout;
            a.exact = 1;
            a.only_flagged = 1;
            launch_scan8_exact(dix, a, s);
        } else {
            a.kk = (int)kout;
            a.exact = 1;
            launch_scan8_exact(dix, a, s);
            if (allp) VGPU_HIP(hipEventRecord(ev[4], s));
            if (scanp) VGPU_HIP(hipEventRecord(ws->sev[4 * ci + 1], s));
        }
        if (allp) VGPU_HIP(hipEventRecord(ev[5], s));
        const uint32_t* vout = nullptr;  // rows already final
        const float* dout = nullptr;
        size_t kin = kout;
        if (pl.pool) {
            launch_rerank(dix, w.qn, (int)nc, w.vidx, (int)kout, (int)k, w.vidx2, w.dist2, s);
            vout = w.vidx2;
            dout = w.dist2;
            kin = k;
        }
        if (allp) VGPU_HIP(hipEventRecord(ev[6], s));
        launch_finish(vout, dout, d_doc_ids.p, (int)nc, (int)kin, (int)k, d_ids + q0 * k, d_dists + q0 * k,
                      w.qstat, counters, flag_count, cflag_count, s, w.qbad);
        if (allp) VGPU_HIP(hipEventRecord(ev[7], s));
        VGPU_HIP(hipGetLastError());
        if (allp) {
            VGPU_HIP(hipEventSynchronize(ev[7]));
            float ms;
            for (int i = 0; i < 7; i++) {
                VGPU_HIP(hipEventElapsedTime(&ms, ev[i], ev[i + 1]));
                t[i] += ms;
            }
            if (pl.t2) {  // the scan phase less the table pre-pass
                VGPU_HIP(hipEventElapsedTime(&ms, ev[3], ev[8]));
                t[3] -= ms;
                t_table += ms;
            }
        }
    }
    if (!ws) {
        complete_noalloc(w, s);
        return;
    }
    unsigned long long* h_scal = ws->h_scal;
    VGPU_HIP(hipMemcpyAsync(h_scal, w.scal, kScalWords * sizeof(unsigned long long), hipMemcpyDeviceToHost, s));
    VGPU_HIP(hipStreamSynchronize(s));
    check_nonfinite(h_scal[kBadWord]);
    if (scanp) {  // the scan kernels of every chunk, read after the final wait
        for (size_t c = 0; c < ci; c++) {
            float ms;
            VGPU_HIP(hipEventElapsedTime(&ms, ws->sev[4 * c], ws->sev[4 * c + 1]));
            t[3] += ms;
            if (pl.t2) {
                VGPU_HIP(hipEventElapsedTime(&ms, ws->sev[4 * c + 2], ws->sev[4 * c + 3]));
                t_table += ms;
            }
        }
    }
    unsigned long long cnt[NUM_SCAN_COUNTERS];
    for (int i = 0; i < NUM_SCAN_COUNTERS; i++) cnt[i] = h_scal[i * COUNTER_STRIDE];
    const unsigned int ovf = reinterpret_cast<const unsigned int*>(h_scal + kOverflowWord)[0] +
                             (unsigned int)h_scal[NUM_SCAN_COUNTERS * COUNTER_STRIDE];
    st->ms_normalize = t[0];
    st->ms_coarse = t[1];
    st->ms_select = t[2];
    st->ms_scan = t[3];
    st->ms_fallback = t[4];
    st->ms_rerank = t[5];
    st->ms_table = t_table;
    st->ms_total = t[0] + t[1] + t[2] + t[3] + t[4] + t[5] + t[6] + t_table;
    st->candidates = cnt[0];
    st->fallback_queries = (uint32_t)cnt[1];
    st->fast_flushes = cnt[2];
    st->fast_appends = cnt[3];
    st->fallback_ties = (uint32_t)cnt[4];
    st->fast_retries = (uint32_t)cnt[5];
    st->coarse_overflow = ovf;
    st->scan_bytes = K == 16 ? cnt[0] * (uint64_t)(M / 2 + 4) : cnt[0] * (uint64_t)(M + 4);
}

void IvfpqIndex::search_device(const float* d_q, size_t nq, size_t k, size_t nprobe, size_t pool,
                               int64_t* d_ids, float* d_dists, hipStream_t s) {
    if (!built) throw Error(VGPU_ERR_NOT_BUILT, "IVF-PQ index: search before build");
    vgpu_search_stats st{};
    st.nq = (uint32_t)nq;
    if (nq == 0 || k == 0) {
        std::lock_guard<std::mutex> lk(stats_mu);
        stats = st;
        return;
    }
    const SearchPlan pl = plan_search(nq, k, nprobe, pool);
    WsLease ws(*this, take_ws());
    if (!s) s = ws->stream;
    ws.used = s;
    const size_t bytes = ws_layout(pl, nullptr, nullptr);
    ws->arena.reserve(bytes);
    WsPtrs w;
    ws_layout(pl, ws->arena.p, &w);
    run_search(d_q, nq, pl, w, d_ids, d_dists, s, ws.ws.get(), &st);
    std::lock_guard<std::mutex> lk(stats_mu);
    stats = st;
}

void IvfpqIndex::search_device_in(const float* d_q, size_t nq, size_t k, size_t nprobe, size_t pool,
                                  int64_t* d_ids, float* d_dists, hipStream_t s, uint8_t* arena,
                                  size_t bytes) {
    if (!built) throw Error(VGPU_ERR_NOT_BUILT, "IVF-PQ index: search before build");
    if (nq == 0 || k == 0) return;
    SearchPlan pl = plan_search(nq, k, nprobe, pool);
    // the largest chunk whose arena fits the caller's bytes
    size_t lo = 0, hi = pl.chunk;
    while (lo < hi) {
        const size_t mid = (lo + hi + 1) / 2;
        SearchPlan t = pl;
        t.chunk = mid;
        if (ws_layout(t, nullptr, nullptr) <= bytes) lo = mid;
        else hi = mid - 1;
    }
    if (lo == 0) {
        SearchPlan one = pl;
        one.chunk = 1;
        throw Error(VGPU_ERR_INVALID_PARAMETER,
                    "allocation-free search needs " + std::to_string(ws_layout(one, nullptr, nullptr)) +
                        " bytes of scratch for one query at this shape; the scratch holds " +
                        std::to_string(bytes));
    }
    pl.chunk = lo;
    WsPtrs w;
    ws_layout(pl, arena, &w);
    run_search(d_q, nq, pl, w, d_ids, d_dists, s ? s : stream, nullptr, nullptr);
}

// search.rs:857-884: codes of insertion index idx decoded (pq.rs:284-290;
// OPQ: opq.rs:134-139, R^T v summed in order with one rounding per product
// and per sum, opq.rs:194-204), plus the centroid of the list holding idx
// (found by a scan of the lists, as cluster_of does).
void IvfpqIndex::reconstruct(size_t idx, float* out) const {
    if (!built) throw Error(VGPU_ERR_INVALID_PARAMETER, "index must be built before reconstruct");
    if (idx >= n())
        throw Error(VGPU_ERR_INVALID_PARAMETER, "vector index " + std::to_string(idx) +
                                                    " out of range (num_vectors = " + std::to_string(n()) + ")");
    size_t pos = 0;
    while (pos < list_ids.size() && list_ids[pos] != (uint32_t)idx) pos++;
    if (pos == list_ids.size())
        throw Error(VGPU_ERR_DEVICE, "vector index " + std::to_string(idx) + " is not in any inverted list");
    const size_t l = std::upper_bound(offsets.begin(), offsets.end(), (uint64_t)pos) - offsets.begin() - 1;
    std::vector<float> dec(d);
    for (size_t m = 0; m < M; m++) {
        const uint8_t c = codes[idx * M + m];
        std::memcpy(&dec[m * ds], &codebooks[(m * K + c) * ds], ds * sizeof(float));
    }
    if (!rotation.empty()) {
        std::vector<float> r(d);
        for (size_t i = 0; i < d; i++) {
            float sum = 0.0f;
            for (size_t j = 0; j < d; j++) sum += rotation[j * d + i] * dec[j];  // -ffp-contract=off: no FMA
            r[i] = sum;
        }
        dec.swap(r);
    }
    for (size_t i = 0; i < d; i++) out[i] = dec[i] + centroids[l * d + i];
}

// search.rs:1552-1577 by the reference's categories over the host mirror,
// plus the device buffers of the index and its pooled search workspaces.
vgpu_memory_report IvfpqIndex::memory_usage() {
    vgpu_memory_report r{};
    r.vectors_bytes = vectors.size() * sizeof(float);
    r.quantized_bytes = codes.size() + codebooks.size() * sizeof(float) + rotation.size() * sizeof(float);
    r.metadata_bytes = doc_ids.size() * sizeof(uint32_t) + centroids.size() * sizeof(float) +
                       offsets.size() * sizeof(uint64_t) + list_ids.size() * sizeof(uint32_t) +
                       list_mask.size() * sizeof(uint64_t);
    size_t dev = d_centroids.bytes() + d_codebooks.bytes() + d_bias.bytes() + d_vectors.bytes() +
                 d_rotation.bytes() + d_cb16.bytes() + d_offsets.bytes() + d_list_ids.bytes() +
                 d_doc_ids.bytes() + d_pack_off.bytes() + d_codes.bytes() + d_packed.bytes() +
                 d_tblocks.bytes() + d_tblk_off.bytes() + d_ecat.bytes() + b_cb16.bytes() + b_dots.bytes() +
                 b_cflag_list.bytes() + b_cflag_count.bytes() +
                 b_overflow.bytes();
    {
        std::lock_guard<std::mutex> lk(pool_mu);
        for (const auto& w : ws_pool)
            dev += w->arena.bytes() + w->q.bytes() + w->odist.bytes() + w->ids.bytes() + w->slots.bytes() +
                   w->want.bytes() + w->fqn.bytes() + w->fdist.bytes() + w->frres.bytes() + w->fvidx.bytes() +
                   w->gprobe.bytes();
    }
    r.device_bytes = dev;
    return r;
}

void IvfpqIndex::search_host(const float* q, size_t nq, size_t k, size_t nprobe, size_t pool,
                             int64_t* ids, float* dists) {
    for (size_t i = 0; i < nq * d; i++)
        if (!std::isfinite(q[i])) throw Error(VGPU_ERR_INVALID_PARAMETER, "query contains a non-finite value");
    if (!built) throw Error(VGPU_ERR_NOT_BUILT, "IVF-PQ index: search before build");
    if (nq == 0 || k == 0) return;
    const SearchPlan pl = plan_search(nq, k, nprobe, pool);
    WsLease ws(*this, take_ws());
    hipStream_t s = ws->stream;
    ws->q.upload(q, nq * d, s);
    ws->ids.reserve(nq * k);
    ws->odist.reserve(nq * k);
    ws->arena.reserve(ws_layout(pl, nullptr, nullptr));
    WsPtrs w;
    ws_layout(pl, ws->arena.p, &w);
    vgpu_search_stats st{};
    st.nq = (uint32_t)nq;
    run_search(ws->q.p, nq, pl, w, ws->ids.p, ws->odist.p, s, ws.ws.get(), &st);
    VGPU_HIP(hipMemcpyAsync(ids, ws->ids.p, nq * k * sizeof(int64_t), hipMemcpyDeviceToHost, s));
    VGPU_HIP(hipMemcpyAsync(dists, ws->odist.p, nq * k * sizeof(float), hipMemcpyDeviceToHost, s));
    VGPU_HIP(hipStreamSynchronize(s));
    std::lock_guard<std::mutex> lk(stats_mu);
    stats = st;
}

void IvfpqIndex::search_host_probed(const float* q, size_t nq, size_t P, const uint32_t* probes,
                                    size_t k, int64_t* ids, float* dists) {
    if (!built) throw Error(VGPU_ERR_NOT_BUILT, "IVF-PQ index: search before build");
    if (nq == 0 || k == 0) return;
    if (P > L) throw Error(VGPU_ERR_INVALID_PARAMETER, "more probes than lists");
    for (size_t i = 0; i < nq * P; i++)
        if (probes[i] >= L) throw Error(VGPU_ERR_INVALID_PARAMETER, "probe list out of range");
    const SearchPlan pl = plan_search(nq, k, P, 0);
    WsLease ws(*this, take_ws());
    hipStream_t s = ws->stream;
    ws->q.upload(q, nq * d, s);
    if (P) ws->gprobe.upload(probes, nq * P, s);
    else ws->gprobe.reserve(1);
    ws->ids.reserve(nq * k);
    ws->odist.reserve(nq * k);
    ws->arena.reserve(ws_layout(pl, nullptr, nullptr));
    WsPtrs w;
    ws_layout(pl, ws->arena.p, &w);
    vgpu_search_stats st{};
    st.nq = (uint32_t)nq;
    run_search(ws->q.p, nq, pl, w, ws->ids.p, ws->odist.p, s, ws.ws.get(), &st, ws->gprobe.p);
    VGPU_HIP(hipMemcpyAsync(ids, ws->ids.p, nq * k * sizeof(int64_t), hipMemcpyDeviceToHost, s));
    VGPU_HIP(hipMemcpyAsync(dists, ws->odist.p, nq * k * sizeof(float), hipMemcpyDeviceToHost, s));
    VGPU_HIP(hipStreamSynchronize(s));
    std::lock_guard<std::mutex> lk(stats_mu);
    stats = st;
}

void IvfpqIndex::probe_host(const float* q, size_t nq, size_t nprobe, uint32_t* lists) {
    if (!built) throw Error(VGPU_ERR_NOT_BUILT, "IVF-PQ index: probe before build");
    const size_t P = std::min(nprobe, L);
    if (nq == 0 || P == 0) return;
    SearchPlan pl = plan_search(nq, 1, P, 0);
    WsLease ws(*this, take_ws());
    hipStream_t s = ws->stream;
    ws->q.upload(q, nq * d, s);
    ws->arena.reserve(ws_layout(pl, nullptr, nullptr));
    WsPtrs w;
    ws_layout(pl, ws->arena.p, &w);
    launch_zero_words(w.scal, kScalWords, s);
    uint32_t* cflag_count = reinterpret_cast<uint32_t*>(w.scal + kCFlagWord);
    for (size_t q0 = 0; q0 < nq; q0 += pl.chunk) {
        const size_t nc = std::min(pl.chunk, nq - q0);
        launch_zero_words(reinterpret_cast<unsigned long long*>(cflag_count), 1, s);
        coarse_probe(ws->q.p + q0 * d, nc, P, pl, w, s, nullptr, true);
        VGPU_HIP(hipMemcpyAsync(lists + q0 * P, w.probe, nc * P * sizeof(uint32_t), hipMemcpyDeviceToHost, s));
    }
    VGPU_HIP(hipGetLastError());
    VGPU_HIP(hipStreamSynchronize(s));
}

}  // namespace vgpu

namespace vgpu {

// ---- search_with_filter (search.rs:1407-1549) ----------------------------

// IVFPQIndex::with_filtering (search.rs:413-435) makes a filtering index at
// construction; here it is switched on before the lists exist.
void IvfpqIndex::enable_filtering() {
    if (built)
        throw Error(VGPU_ERR_ALREADY_BUILT, "filtering must be enabled before build (IVFPQIndex::with_filtering)");
    filtering = true;
}

// add_metadata (search.rs:439-475), the filter field only: 0..63, or -1 for
// metadata without the field (such a document never matches).
void IvfpqIndex::set_category(uint32_t doc_id, int cat) {
    if (!filtering)
        throw Error(VGPU_ERR_UNSUPPORTED,
                    "filtered search: rebuild the index with IVFPQIndex::with_filtering()");
    if (cat < -1 || cat > 63)
        throw Error(VGPU_ERR_INVALID_PARAMETER, "category ID " + std::to_string(cat) +
                                                    " exceeds bitmask limit of 63; use an integer in 0..63");
    doc_cat[doc_id] = cat;
    cat_dirty = true;
}

// search.rs:626-648: list l's bitmask holds the categories of its members
// when the lists are built (metadata added later does not change it).
void IvfpqIndex::snapshot_list_masks() {
    list_mask.assign(L, 0ull);
    cat_dirty = true;
    if (!filtering || doc_cat.empty()) return;
    for (size_t l = 0; l < L; l++)
        for (uint64_t p = offsets[l]; p < offsets[l + 1]; p++) {
            const auto it = doc_cat.find(doc_ids[list_ids[p]]);
            if (it != doc_cat.end() && it->second >= 0) list_mask[l] |= 1ull << it->second;
        }
}

// The current category of every list-major entry (what
// MetadataStore::matches reads, filtering/mod.rs:214-218) and the per-list
// counts the widening test needs.
void IvfpqIndex::refresh_categories(hipStream_t s) {
    std::lock_guard<std::mutex> lk(cat_mu);
    if (!cat_dirty) return;
    const size_t nv = n();
    std::vector<uint8_t> ec(nv, 0xff);
    list_cat_n.assign(L * 64, 0u);
    for (size_t l = 0; l < L; l++)
        for (uint64_t p = offsets[l]; p < offsets[l + 1]; p++) {
            const auto it = doc_cat.find(doc_ids[list_ids[p]]);
            if (it != doc_cat.end() && it->second >= 0) {
                ec[p] = (uint8_t)it->second;
                list_cat_n[l * 64 + (size_t)it->second]++;
            }
        }
    d_ecat.upload(ec.data(), nv, s);
    VGPU_HIP(hipStreamSynchronize(s));
    cat_dirty = false;
}

// The probed lists (nearest first) that carry the query's category are
// scanned; when their members of that category number fewer than k and some
// lists were not probed, every other list carrying it follows in index order
// (search.rs:1486-1545).  Matches are scored with the reference's table
// arithmetic and the k smallest kept (finish_top_k_by_distance, :64-75).
void IvfpqIndex::search_filtered(const float* q, size_t nq, size_t k, const int* cats, int64_t* ids,
                                 float* dists) {
    if (!built) throw Error(VGPU_ERR_NOT_BUILT, "IVF-PQ index: search before build");
    if (!filtering)
        throw Error(VGPU_ERR_INVALID_PARAMETER, "filter field doesn't match index filter field (None)");
    for (size_t i = 0; i < nq; i++)
        if (cats[i] < 0 || cats[i] > 63)
            throw Error(VGPU_ERR_INVALID_PARAMETER, "category ID " + std::to_string(cats[i]) +
                                                        " exceeds bitmask limit of 63");
    for (size_t i = 0; i < nq * d; i++)
        if (!std::isfinite(q[i])) throw Error(VGPU_ERR_INVALID_PARAMETER, "query contains a non-finite value");
    if (nq == 0 || k == 0) return;
    {
        ScanArgs shape;  // the filtered kernel's LDS: the EXACT table and buffer, no per-list arrays
        shape.kk = (int)k;
        if (scan8_lds_bytes(dix, shape) > 160 * 1024)
            throw Error(VGPU_ERR_UNSUPPORTED, "filtered scan working set exceeds the 160 KiB of LDS per workgroup");
    }
    // probe with the index's nprobe (which may be 0: then every list that
    // carries the category is a widening candidate)
    const SearchPlan pl = plan_search(nq, 1, 0, 0);
    const size_t P = pl.P;
    WsLease ws(*this, take_ws());
    hipStream_t s = ws->stream;
    ws->q.upload(q, nq * d, s);
    ws->arena.reserve(ws_layout(pl, nullptr, nullptr));
    WsPtrs w;
    ws_layout(pl, ws->arena.p, &w);
    ws->fqn.reserve(nq * d);
    std::vector<uint32_t> probes(nq * P);
    launch_zero_words(w.scal, kScalWords, s);
    uint32_t* cflag_count = reinterpret_cast<uint32_t*>(w.scal + kCFlagWord);
    for (size_t q0 = 0; q0 < nq; q0 += pl.chunk) {
        const size_t nc = std::min(pl.chunk, nq - q0);
        launch_zero_words(reinterpret_cast<unsigned long long*>(cflag_count), 1, s);
        coarse_probe(ws->q.p + q0 * d, nc, P, pl, w, s, nullptr, true);
        VGPU_HIP(hipMemcpyAsync(ws->fqn.p + q0 * d, w.qn, nc * d * sizeof(float), hipMemcpyDeviceToDevice, s));
        if (P)
            VGPU_HIP(hipMemcpyAsync(probes.data() + q0 * P, w.probe, nc * P * sizeof(uint32_t),
                                    hipMemcpyDeviceToHost, s));
    }
    VGPU_HIP(hipGetLastError());
    VGPU_HIP(hipStreamSynchronize(s));
    check_labels(probes.data(), nq * P, 1, L, "probed lists");
    refresh_categories(s);
    std::vector<std::vector<uint32_t>> order(nq);
    std::vector<char> probed;
    size_t pmax = 1;
    for (size_t i = 0; i < nq; i++) {
        const uint64_t bit = 1ull << cats[i];
        size_t found = 0;
        for (size_t p = 0; p < P; p++) {
            const uint32_t l = probes[i * P + p];
            if (list_mask[l] & bit) {
                order[i].push_back(l);
                found += list_cat_n[(size_t)l * 64 + (size_t)cats[i]];
            }
        }
        if (found < k && P < L) {
            probed.assign(L, 0);
            for (size_t p = 0; p < P; p++) probed[probes[i * P + p]] = 1;
            for (size_t l = 0; l < L; l++)
                if (!probed[l] && (list_mask[l] & bit)) order[i].push_back((uint32_t)l);
        }
        pmax = std::max(pmax, order[i].size());
    }
    std::vector<uint32_t> slots(nq * pmax, 0xffffffffu);
    std::vector<uint8_t> want(nq);
    for (size_t i = 0; i < nq; i++) {
        std::copy(order[i].begin(), order[i].end(), slots.begin() + i * pmax);
        want[i] = (uint8_t)cats[i];
    }
    ws->slots.upload(slots.data(), nq * pmax, s);
    ws->want.upload(want.data(), nq, s);
    ws->fvidx.reserve(nq * k);
    ws->fdist.reserve(nq * k);
    ws->ids.reserve(nq * k);
    ws->odist.reserve(nq * k);
    // OPQ rotates every (query, slot) residual first; queries go in chunks that
    // bound that buffer at rres_limit floats (a widened query has up to L slots).
    const bool opq = !rotation.empty();
    const size_t chunk = opq ? std::max<size_t>(1, rres_limit / (pmax * d)) : nq;
    if (opq) ws->frres.reserve(std::min(chunk, nq) * pmax * d);
    for (size_t q0 = 0; q0 < nq; q0 += chunk) {
        const size_t nc = std::min(chunk, nq - q0);
        ScanArgs a;
        a.qn = ws->fqn.p + q0 * d;
        a.qnorm = nullptr;  // not read by the filtered kernel
        a.probe = ws->slots.p + q0 * pmax;
        a.nq = (int)nc;
        a.P = (int)pmax;
        a.kout = (int)k;
        a.kk = (int)k;
        a.exact = 1;
        a.out_vidx = ws->fvidx.p + q0 * k;
        a.out_dist = ws->fdist.p + q0 * k;
        if (opq) {
            rotate_slots(a.qn, nc, pmax, a.probe, ws->frres.p, s);
            a.rres = ws->frres.p;
        }
        launch_scan8_filtered(dix, a, d_ecat.p, ws->want.p + q0, s);
    }
    launch_finish(ws->fvidx.p, ws->fdist.p, d_doc_ids.p, (int)nq, (int)k, (int)k, ws->ids.p, ws->odist.p,
                  nullptr, nullptr, nullptr, nullptr, s);
    VGPU_HIP(hipGetLastError());
    VGPU_HIP(hipMemcpyAsync(ids, ws->ids.p, nq * k * sizeof(int64_t), hipMemcpyDeviceToHost, s));
    VGPU_HIP(hipMemcpyAsync(dists, ws->odist.p, nq * k * sizeof(float), hipMemcpyDeviceToHost, s));
    VGPU_HIP(hipStreamSynchronize(s));
}

}  // namespace vgpu
