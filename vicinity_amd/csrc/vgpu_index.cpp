// IVF-PQ index object: insert, GPU-assisted build, HBM residency, and the
// batched search pipeline.
//
// Reference: IVFPQIndex src/ivf_pq/search.rs:212-239 (state), add_slice
// :488-512, build_with_training_config :546-787, build_scan_caches :816-848,
// search :1087-1093, search_reranked :1117-1158, search_approx_internal_observed
// :1175-1391; batch shape src/python.rs:744-793.
#include <algorithm>
#include <cmath>
#include <cstring>
#include <numeric>
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
    VGPU_HIP(hipStreamCreate(&stream));
    for (auto& e : ev) VGPU_HIP(hipEventCreate(&e));
}

IvfpqIndex::~IvfpqIndex() {
    if (stream) (void)hipStreamSynchronize(stream);
    if (h_scal) (void)hipHostFree(h_scal);
    for (auto& e : ev)
        if (e) (void)hipEventDestroy(e);
    for (auto& e : sev)
        if (e) (void)hipEventDestroy(e);
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
        const int cap = coarse_fused_cap(1);
        w_cb16.reserve(coarse_bf16_pack_chunks((int)k, (int)d));
        w_cand.reserve(chunk * cap);
        w_cand_n.reserve(chunk);
        w_cflag_list.reserve(chunk);
        w_cflag_count.reserve(1);
        w_overflow.reserve(1);
        VGPU_HIP(hipMemsetAsync(w_overflow.p, 0, sizeof(unsigned int), s));
        launch_coarse_bf16_pack(d_cent, (int)k, (int)d, w_cb16.p, s);
        for (size_t q0 = 0; q0 < nx; q0 += chunk) {
            const size_t nc = std::min(chunk, nx - q0);
            VGPU_HIP(hipMemsetAsync(w_cflag_count.p, 0, sizeof(uint32_t), s));
            launch_coarse_fused(d_x + q0 * d, (int)nc, (int)d, w_cb16.p, (int)k, cmax, 1, 0, nullptr,
                                nullptr, w_cand.p, w_cand_n.p, s);
            launch_coarse_topp(w_cand.p, w_cand_n.p, 1, d_x + q0 * d, d_cent, (int)nc, (int)k, (int)d,
                               d_assign + q0, w_cflag_list.p, w_cflag_count.p, s);
            launch_coarse_exact_flagged(d_x + q0 * d, d_norms + q0, d_cent, (int)nc, (int)k, (int)d, 1,
                                        cmax, d_assign + q0, w_overflow.p, w_cflag_list.p,
                                        w_cflag_count.p, s);
        }
        VGPU_HIP(hipGetLastError());
        return;
    }
    size_t chunk = std::max<size_t>(1, std::min<size_t>(nx, ((size_t)1 << 28) / std::max<size_t>(k, 1)));
    chunk = std::min<size_t>(chunk, (size_t)1 << 20);  // grid.y of the GEMM stays < 65536
    w_dots.reserve(chunk * k);
    w_cflag_list.reserve(chunk);
    w_cflag_count.reserve(1);
    w_overflow.reserve(1);
    VGPU_HIP(hipMemsetAsync(w_overflow.p, 0, sizeof(unsigned int), s));
    for (size_t q0 = 0; q0 < nx; q0 += chunk) {
        size_t nc = std::min(chunk, nx - q0);
        launch_coarse_dots(d_x + q0 * d, d_cent, w_dots.p, (int)nc, (int)k, (int)d, s);
        VGPU_HIP(hipMemsetAsync(w_cflag_count.p, 0, sizeof(uint32_t), s));
        launch_coarse_select(w_dots.p, d_x + q0 * d, d_norms + q0, d_cent, (int)nc, (int)k, (int)d, 1,
                             cmax, d_assign + q0, w_overflow.p, w_cflag_list.p, w_cflag_count.p, s);
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
    std::vector<double> sums(ke * d);
    std::vector<uint64_t> counts(ke);
    const bool gpu_update = d <= 256;
    dc.upload(cent.data(), ke * d, stream);
    for (size_t it = 0; it < max_iter; it++) {
        float cmax = 0.0f;
        for (size_t c = 0; c < ke; c++) cmax = std::max(cmax, row_norm_bound(&cent[c * d], d));
        if (!gpu_update) dc.upload(cent.data(), ke * d, stream);
        assign_cosine(dx.p, dn.p, nt, dc.p, ke, cmax, da.p, stream);
        VGPU_HIP(hipMemcpyAsync(assign.data(), da.p, nt * sizeof(uint32_t), hipMemcpyDeviceToHost, stream));
        VGPU_HIP(hipStreamSynchronize(stream));
        if (it > 0 && assign == prev) break;
        if (gpu_update) {
            launch_kmeans_update(dx.p, (int)nt, (int)d, (int)d, 1, da.p, false, (int)ke, nullptr, true, dc.p,
                                 stream);
            VGPU_HIP(hipGetLastError());
            VGPU_HIP(hipMemcpyAsync(cent.data(), dc.p, ke * d * sizeof(float), hipMemcpyDeviceToHost, stream));
            VGPU_HIP(hipStreamSynchronize(stream));
            prev.swap(assign);
            continue;
        }
        std::fill(sums.begin(), sums.end(), 0.0);
        std::fill(counts.begin(), counts.end(), 0);
        for (size_t i = 0; i < nt; i++) {
            double* sc = &sums[(size_t)assign[i] * d];
            const float* xi = &x[i * d];
            for (size_t j = 0; j < d; j++) sc[j] += (double)xi[j];
            counts[assign[i]]++;
        }
        for (size_t c = 0; c < ke; c++) {
            if (!counts[c]) continue;
            float* cc = &cent[c * d];
            for (size_t j = 0; j < d; j++) cc[j] = (float)(sums[c * d + j] / (double)counts[c]);
            normalize_row(cc, d, cc);
        }
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
    std::vector<double> sums(Ke * ds);
    std::vector<uint64_t> counts(Ke);
    const bool gpu_update = ds <= 256;
    dcb.upload(codebooks.data(), codebooks.size(), stream);
    for (size_t it = 0; it < max_iter; it++) {
        if (!gpu_update) dcb.upload(codebooks.data(), codebooks.size(), stream);
        launch_encode(dres.p, (int)nt, (int)d, nullptr, nullptr, dcb.p, (int)M, (int)Ke, (int)ds,
                      dcodes.p, stream);
        VGPU_HIP(hipGetLastError());
        VGPU_HIP(hipMemcpyAsync(cur.data(), dcodes.p, nt * M, hipMemcpyDeviceToHost, stream));
        VGPU_HIP(hipStreamSynchronize(stream));
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
            std::fill(sums.begin(), sums.end(), 0.0);
            std::fill(counts.begin(), counts.end(), 0);
            for (size_t i = 0; i < nt; i++) {
                uint8_t c = cur[i * M + m];
                const float* xi = &res[i * d + m * ds];
                for (size_t j = 0; j < ds; j++) sums[c * ds + j] += (double)xi[j];
                counts[c]++;
            }
            for (size_t c = 0; c < Ke; c++) {
                if (!counts[c]) continue;
                for (size_t j = 0; j < ds; j++)
                    codebooks[(m * Ke + c) * ds + j] = (float)(sums[c * ds + j] / (double)counts[c]);
            }
        }
        if (!any) break;
        if (gpu_update) {
            dactive.upload(active.data(), M, stream);
            launch_kmeans_update(dres.p, (int)nt, (int)d, (int)ds, (int)M, dcodes.p, true, (int)Ke, dactive.p,
                                 false, dcb.p, stream);
            VGPU_HIP(hipGetLastError());
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

    // Lists: insertion order inside a list (search.rs:624-657).
    offsets.assign(L + 1, 0);
    for (size_t i = 0; i < n; i++) offsets[assign[i] + 1]++;
    for (size_t l = 0; l < L; l++) offsets[l + 1] += offsets[l];
    list_ids.resize(n);
    {
        std::vector<uint64_t> fill(offsets.begin(), offsets.end() - 1);
        for (size_t i = 0; i < n; i++) list_ids[fill[assign[i]]++] = (uint32_t)i;
    }

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
        dix.tblocks = nullptr;
        dix.tblk_off = nullptr;
    } else {
        d_bias.reserve(n);
        dix.bias = d_bias.p;
        launch_bias(dix, d_bias.p, stream);
        std::vector<uint32_t> toff(L + 1, 0);
        for (size_t l = 0; l < L; l++)
            toff[l + 1] = toff[l] + (uint32_t)((offsets[l + 1] - offsets[l] + 15) / 16);
        const size_t tbytes = ((size_t)toff[L] + 1) * TBLK_BYTES(M);  // + one block of slack
        if (scan8_fast_blocks_supported((int)M, (int)K, (int)ds) && tbytes < ((size_t)1 << 31)) {
            d_tblk_off.upload(toff.data(), L + 1, stream);
            d_tblocks.reserve(tbytes);
            dix.tblk_off = d_tblk_off.p;
            dix.tblocks = d_tblocks.p;
            dix.tblk_bytes = (uint32_t)tbytes;
            launch_tblocks(dix, d_tblocks.p, stream);
        } else {
            d_tblocks.release();
            d_tblk_off.release();
        }
    }
    VGPU_HIP(hipGetLastError());
    VGPU_HIP(hipStreamSynchronize(stream));
}

// Word offsets in the per-call scalar buffer (64-byte lines apart).
static constexpr size_t kOverflowWord = (NUM_SCAN_COUNTERS + 1) * COUNTER_STRIDE;
static constexpr size_t kFlagWord = kOverflowWord + 8;
static constexpr size_t kCFlagWord = kFlagWord + 8;
static constexpr size_t kScalWords = kCFlagWord + 8;

static int fast_keep(size_t kout) {
    int kk = 1;
    while ((size_t)kk < kout + 16) kk <<= 1;
    return std::max(kk, 32);
}

void IvfpqIndex::search_device(const float* d_q, size_t nq, size_t k, size_t nprobe, size_t pool,
                               int64_t* d_ids, float* d_dists, hipStream_t s) {
    if (!built) throw Error(VGPU_ERR_NOT_BUILT, "IVF-PQ index: search before build");
    if (!s) s = stream;
    stats = vgpu_search_stats{};
    stats.nq = (uint32_t)nq;
    if (nq == 0 || k == 0) return;
    if (pool && !has_vectors)
        throw Error(VGPU_ERR_UNSUPPORTED, "search_reranked after compact(): raw vectors were dropped");
    size_t P = nprobe ? nprobe : params.nprobe;
    P = std::min(P, L);
    const size_t kout = pool ? std::max(pool, k) : k;
    if (kout > 2048) throw Error(VGPU_ERR_INVALID_PARAMETER, "k / rerank_pool above 2048 is not supported");
    if (P > 1024) throw Error(VGPU_ERR_INVALID_PARAMETER, "nprobe above 1024 is not supported");
    {
        ScanArgs probe_shape;
        probe_shape.P = (int)P;
        probe_shape.kout = (int)kout;
        probe_shape.kk = K == 16 ? (int)kout : fast_keep(kout);
        size_t lds = K == 16 ? fastscan_lds_bytes(dix, probe_shape)
                             : std::max(scan8_fast_lds_bytes(dix, probe_shape),
                                        scan8_lds_bytes(dix, probe_shape));
        if (lds > 160 * 1024)
            throw Error(VGPU_ERR_UNSUPPORTED, "scan working set of " + std::to_string(lds) +
                                                  " bytes exceeds the 160 KiB of LDS per workgroup");
    }
    if (P == 0) {  // no probed list: every row is padding
        launch_finalize(nullptr, nullptr, nullptr, (int)nq, 0, (int)k, d_ids, d_dists, s);
        VGPU_HIP(hipGetLastError());
        VGPU_HIP(hipStreamSynchronize(s));
        return;
    }
    const bool opq = !rotation.empty();
    size_t chunk = std::max<size_t>(1, std::min<size_t>(nq, ((size_t)1 << 28) / L));
    chunk = std::min<size_t>(chunk, 65536);
    if (opq) chunk = std::max<size_t>(1, std::min<size_t>(chunk, ((size_t)1 << 28) / (P * d)));
    w_qn.reserve(chunk * d);
    w_qnorm.reserve(chunk);
    const bool fused = coarse_fused_supported((int)d, (int)P);
    if (fused) {
        w_cand.reserve(chunk * coarse_fused_cap((int)P));
        w_cand_n.reserve(chunk);
    } else {
        w_dots.reserve(chunk * L);
    }
    w_cflag_list.reserve(chunk);
    w_probe.reserve(chunk * P);
    w_vidx.reserve(chunk * kout);
    w_dist.reserve(chunk * kout);
    w_vidx2.reserve(chunk * k);
    w_dist2.reserve(chunk * k);
    w_qstat.reserve(chunk * QSTAT_WORDS);
    w_flag_list.reserve(chunk);
    // Per-call device scalars in one buffer, cleared by one memset: counter i
    // at word i * COUNTER_STRIDE, then the overflow count and the two
    // flag-list lengths, each on a cache line of its own.
    w_scal.reserve(kScalWords);
    if (!h_scal) VGPU_HIP(hipHostMalloc((void**)&h_scal, kScalWords * sizeof(unsigned long long)));
    unsigned long long* counters = w_scal.p;
    unsigned int* overflow = reinterpret_cast<unsigned int*>(w_scal.p + kOverflowWord);
    uint32_t* flag_count = reinterpret_cast<uint32_t*>(w_scal.p + kFlagWord);
    uint32_t* cflag_count = reinterpret_cast<uint32_t*>(w_scal.p + kCFlagWord);
    VGPU_HIP(hipMemsetAsync(w_scal.p, 0, kScalWords * sizeof(unsigned long long), s));
    float t[7] = {0, 0, 0, 0, 0, 0, 0};
    const bool allp = profiling == 1, scanp = profiling == 2;
    if (scanp) {
        const size_t need_ev = 2 * ((nq + chunk - 1) / chunk);
        while (sev.size() < need_ev) {
            hipEvent_t e;
            VGPU_HIP(hipEventCreate(&e));
            sev.push_back(e);
        }
    }
    size_t ci = 0;  // chunk index
    for (size_t q0 = 0; q0 < nq; q0 += chunk, ci++) {
        const size_t nc = std::min(chunk, nq - q0);
        if (allp) VGPU_HIP(hipEventRecord(ev[0], s));
        if (fused) {
            // normalise + two bf16x3 MFMA passes (ms_coarse), exact top-P of the
            // candidates and the rare exact fallback (ms_select)
            if (allp) VGPU_HIP(hipEventRecord(ev[1], s));
            launch_coarse_fused(d_q + q0 * d, (int)nc, (int)d, dix.cb16, (int)L, dix.cmax, (int)P, 1,
                                w_qn.p, w_qnorm.p, w_cand.p, w_cand_n.p, s);
            if (allp) VGPU_HIP(hipEventRecord(ev[2], s));
            launch_coarse_topp(w_cand.p, w_cand_n.p, (int)P, w_qn.p, d_centroids.p, (int)nc, (int)L, (int)d,
                               w_probe.p, w_cflag_list.p, cflag_count, s);
            launch_coarse_exact_flagged(w_qn.p, w_qnorm.p, d_centroids.p, (int)nc, (int)L, (int)d, (int)P,
                                        dix.cmax, w_probe.p, overflow, w_cflag_list.p, cflag_count, s);
        } else {
            launch_normalize(d_q + q0 * d, w_qn.p, w_qnorm.p, (int)nc, (int)d, s);
            if (allp) VGPU_HIP(hipEventRecord(ev[1], s));
            launch_coarse_dots(w_qn.p, d_centroids.p, w_dots.p, (int)nc, (int)L, (int)d, s);
            if (allp) VGPU_HIP(hipEventRecord(ev[2], s));
            launch_coarse_select(w_dots.p, w_qn.p, w_qnorm.p, d_centroids.p, (int)nc, (int)L, (int)d,
                                 (int)P, dix.cmax, w_probe.p, overflow, w_cflag_list.p, cflag_count, s);
        }
        // OPQ: the rotated residual of every (query, probe) slot (opq.rs:120-123),
        // timed with the selection
        const float* rres = opq ? rotate_slots(w_qn.p, nc, P, w_probe.p, s) : nullptr;
        if (allp) VGPU_HIP(hipEventRecord(ev[3], s));
        // scan-only timing: the FAST kernel's dispatch records the two events
        // itself; the other scan kernels are bracketed by marker events
        const bool scan_fast = K != 16 && mode == VGPU_MODE_FAST && !opq;
        if (scanp && !scan_fast) VGPU_HIP(hipEventRecord(sev[2 * ci], s));
        ScanArgs a;
        a.qn = w_qn.p;
        a.qnorm = w_qnorm.p;
        a.probe = w_probe.p;
        a.nq = (int)nc;
        a.P = (int)P;
        a.kout = (int)kout;
        a.qstat = w_qstat.p;
        a.flag_list = w_flag_list.p;
        a.flag_count = flag_count;
        a.out_vidx = w_vidx.p;
        a.out_dist = w_dist.p;
        a.rres = rres;
        if (K == 16) {
            a.kk = (int)kout;
            launch_fastscan(dix, a, s);
            if (allp) VGPU_HIP(hipEventRecord(ev[4], s));
            if (scanp) VGPU_HIP(hipEventRecord(sev[2 * ci + 1], s));
        } else if (mode == VGPU_MODE_FAST && !opq) {
            a.kk = fast_keep(kout);
            a.exact = 0;
            launch_scan8_fast(dix, a, s, scanp ? sev[2 * ci] : nullptr, scanp ? sev[2 * ci + 1] : nullptr);
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
            if (scanp) VGPU_HIP(hipEventRecord(sev[2 * ci + 1], s));
        }
        if (allp) VGPU_HIP(hipEventRecord(ev[5], s));
        const uint32_t* vout = w_vidx.p;
        const float* dout = w_dist.p;
        size_t kin = kout;
        if (pool) {
            launch_rerank(dix, w_qn.p, (int)nc, w_vidx.p, (int)kout, (int)k, w_vidx2.p, w_dist2.p, s);
            vout = w_vidx2.p;
            dout = w_dist2.p;
            kin = k;
        }
        if (allp) VGPU_HIP(hipEventRecord(ev[6], s));
        launch_finish(vout, dout, d_doc_ids.p, (int)nc, (int)kin, (int)k, d_ids + q0 * k,
                      d_dists + q0 * k, w_qstat.p, counters, flag_count, cflag_count, s);
        if (allp) VGPU_HIP(hipEventRecord(ev[7], s));
        VGPU_HIP(hipGetLastError());
        if (allp) {
            VGPU_HIP(hipEventSynchronize(ev[7]));
            float ms;
            for (int i = 0; i < 7; i++) {
                VGPU_HIP(hipEventElapsedTime(&ms, ev[i], ev[i + 1]));
                t[i] += ms;
            }
        }
    }
    VGPU_HIP(hipMemcpyAsync(h_scal, w_scal.p, kScalWords * sizeof(unsigned long long),
                            hipMemcpyDeviceToHost, s));
    VGPU_HIP(hipStreamSynchronize(s));
    if (scanp) {  // the scan kernels of every chunk, read after the final wait
        for (size_t c = 0; c < ci; c++) {
            float ms;
            VGPU_HIP(hipEventElapsedTime(&ms, sev[2 * c], sev[2 * c + 1]));
            t[3] += ms;
        }
    }
    unsigned long long cnt[NUM_SCAN_COUNTERS];
    for (int i = 0; i < NUM_SCAN_COUNTERS; i++) cnt[i] = h_scal[i * COUNTER_STRIDE];
    const unsigned int ovf = reinterpret_cast<const unsigned int*>(h_scal + kOverflowWord)[0] +
                             (unsigned int)h_scal[NUM_SCAN_COUNTERS * COUNTER_STRIDE];
    stats.ms_normalize = t[0];
    stats.ms_coarse = t[1];
    stats.ms_select = t[2];
    stats.ms_scan = t[3];
    stats.ms_fallback = t[4];
    stats.ms_rerank = t[5];
    stats.ms_total = t[0] + t[1] + t[2] + t[3] + t[4] + t[5] + t[6];
    stats.candidates = cnt[0];
    stats.fallback_queries = (uint32_t)cnt[1];
    stats.fast_flushes = cnt[2];
    stats.fast_appends = cnt[3];
    stats.fallback_ties = (uint32_t)cnt[4];
    stats.fast_retries = (uint32_t)cnt[5];
    stats.coarse_overflow = ovf;
    stats.scan_bytes = K == 16 ? cnt[0] * (uint64_t)(M / 2 + 4) : cnt[0] * (uint64_t)(M + 4);
}

void IvfpqIndex::search_host(const float* q, size_t nq, size_t k, size_t nprobe, size_t pool,
                             int64_t* ids, float* dists) {
    for (size_t i = 0; i < nq * d; i++)
        if (!std::isfinite(q[i])) throw Error(VGPU_ERR_INVALID_PARAMETER, "query contains a non-finite value");
    if (nq == 0 || k == 0) {
        if (!built) throw Error(VGPU_ERR_NOT_BUILT, "IVF-PQ index: search before build");
        return;
    }
    w_q.upload(q, nq * d, stream);
    w_ids.reserve(nq * k);
    w_odist.reserve(nq * k);
    search_device(w_q.p, nq, k, nprobe, pool, w_ids.p, w_odist.p, stream);
    VGPU_HIP(hipMemcpyAsync(ids, w_ids.p, nq * k * sizeof(int64_t), hipMemcpyDeviceToHost, stream));
    VGPU_HIP(hipMemcpyAsync(dists, w_odist.p, nq * k * sizeof(float), hipMemcpyDeviceToHost, stream));
    VGPU_HIP(hipStreamSynchronize(stream));
}

void IvfpqIndex::probe_host(const float* q, size_t nq, size_t nprobe, uint32_t* lists) {
    if (!built) throw Error(VGPU_ERR_NOT_BUILT, "IVF-PQ index: probe before build");
    size_t P = std::min(nprobe, L);
    if (nq == 0 || P == 0) return;
    if (P > 1024) throw Error(VGPU_ERR_INVALID_PARAMETER, "nprobe above 1024 is not supported");
    w_q.upload(q, nq * d, stream);
    w_qn.reserve(nq * d);
    w_qnorm.reserve(nq);
    w_probe.reserve(nq * P);
    w_overflow.reserve(1);
    VGPU_HIP(hipMemsetAsync(w_overflow.p, 0, sizeof(unsigned int), stream));
    size_t chunk = std::max<size_t>(1, std::min<size_t>(nq, ((size_t)1 << 28) / L));
    w_cflag_list.reserve(chunk);
    w_cflag_count.reserve(1);
    if (coarse_fused_supported((int)d, (int)P)) {
        chunk = std::min<size_t>(nq, (size_t)1 << 20);
        w_cflag_list.reserve(chunk);
        w_cand.reserve(chunk * coarse_fused_cap((int)P));
        w_cand_n.reserve(chunk);
        for (size_t q0 = 0; q0 < nq; q0 += chunk) {
            const size_t nc = std::min(chunk, nq - q0);
            VGPU_HIP(hipMemsetAsync(w_cflag_count.p, 0, sizeof(uint32_t), stream));
            launch_coarse_fused(w_q.p + q0 * d, (int)nc, (int)d, dix.cb16, (int)L, dix.cmax, (int)P, 1,
                                w_qn.p + q0 * d, w_qnorm.p + q0, w_cand.p, w_cand_n.p, stream);
            launch_coarse_topp(w_cand.p, w_cand_n.p, (int)P, w_qn.p + q0 * d, d_centroids.p, (int)nc, (int)L,
                               (int)d, w_probe.p + q0 * P, w_cflag_list.p, w_cflag_count.p, stream);
            launch_coarse_exact_flagged(w_qn.p + q0 * d, w_qnorm.p + q0, d_centroids.p, (int)nc, (int)L,
                                        (int)d, (int)P, dix.cmax, w_probe.p + q0 * P, w_overflow.p,
                                        w_cflag_list.p, w_cflag_count.p, stream);
        }
        VGPU_HIP(hipGetLastError());
        VGPU_HIP(hipMemcpyAsync(lists, w_probe.p, nq * P * sizeof(uint32_t), hipMemcpyDeviceToHost, stream));
        VGPU_HIP(hipStreamSynchronize(stream));
        return;
    }
    w_dots.reserve(chunk * L);
    launch_normalize(w_q.p, w_qn.p, w_qnorm.p, (int)nq, (int)d, stream);
    for (size_t q0 = 0; q0 < nq; q0 += chunk) {
        size_t nc = std::min(chunk, nq - q0);
        launch_coarse_dots(w_qn.p + q0 * d, d_centroids.p, w_dots.p, (int)nc, (int)L, (int)d, stream);
        VGPU_HIP(hipMemsetAsync(w_cflag_count.p, 0, sizeof(uint32_t), stream));
        launch_coarse_select(w_dots.p, w_qn.p + q0 * d, w_qnorm.p + q0, d_centroids.p, (int)nc, (int)L,
                             (int)d, (int)P, dix.cmax, w_probe.p + q0 * P, w_overflow.p,
                             w_cflag_list.p, w_cflag_count.p, stream);
    }
    VGPU_HIP(hipGetLastError());
    VGPU_HIP(hipMemcpyAsync(lists, w_probe.p, nq * P * sizeof(uint32_t), hipMemcpyDeviceToHost, stream));
    VGPU_HIP(hipStreamSynchronize(stream));
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
void IvfpqIndex::refresh_categories() {
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
    d_ecat.upload(ec.data(), nv, stream);
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
    if (k > 2048) throw Error(VGPU_ERR_INVALID_PARAMETER, "k above 2048 is not supported");
    {
        ScanArgs shape;  // the filtered kernel's LDS: the EXACT table and buffer, no per-list arrays
        shape.kk = (int)k;
        if (scan8_lds_bytes(dix, shape) > 160 * 1024)
            throw Error(VGPU_ERR_UNSUPPORTED, "filtered scan working set exceeds the 160 KiB of LDS per workgroup");
    }
    const size_t P = std::min((size_t)params.nprobe, L);
    std::vector<uint32_t> probes(nq * P);
    probe_host(q, nq, params.nprobe, probes.data());  // leaves the normalised queries in w_qn
    refresh_categories();
    std::vector<std::vector<uint32_t>> order(nq);
    std::vector<char> probed;
    size_t pmax = 1;
    for (size_t i = 0; i < nq; i++) {
        const uint64_t bit = 1ull << cats[i];
        size_t found = 0;
        for (size_t p = 0; p < P; p++) {
            const uint32_t l = probes[i * P + p];
            if (l < L && (list_mask[l] & bit)) {
                order[i].push_back(l);
                found += list_cat_n[(size_t)l * 64 + (size_t)cats[i]];
            }
        }
        if (found < k && P < L) {
            probed.assign(L, 0);
            for (size_t p = 0; p < P; p++)
                if (probes[i * P + p] < L) probed[probes[i * P + p]] = 1;
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
    w_probe.upload(slots.data(), nq * pmax, stream);
    w_want.upload(want.data(), nq, stream);
    w_vidx.reserve(nq * k);
    w_dist.reserve(nq * k);
    w_ids.reserve(nq * k);
    w_odist.reserve(nq * k);
    // OPQ rotates every (query, slot) residual first; queries go in chunks that
    // bound that buffer at 2^28 floats (a widened query has up to L slots).
    const bool opq = !rotation.empty();
    const size_t chunk = opq ? std::max<size_t>(1, ((size_t)1 << 28) / (pmax * d)) : nq;
    for (size_t q0 = 0; q0 < nq; q0 += chunk) {
        const size_t nc = std::min(chunk, nq - q0);
        ScanArgs a;
        a.qn = w_qn.p + q0 * d;
        a.qnorm = w_qnorm.p;  // not read by the filtered kernel
        a.probe = w_probe.p + q0 * pmax;
        a.nq = (int)nc;
        a.P = (int)pmax;
        a.kout = (int)k;
        a.kk = (int)k;
        a.exact = 1;
        a.out_vidx = w_vidx.p + q0 * k;
        a.out_dist = w_dist.p + q0 * k;
        if (opq) a.rres = rotate_slots(a.qn, nc, pmax, a.probe, stream);
        launch_scan8_filtered(dix, a, d_ecat.p, w_want.p + q0, stream);
    }
    launch_finish(w_vidx.p, w_dist.p, d_doc_ids.p, (int)nq, (int)k, (int)k, w_ids.p, w_odist.p, nullptr,
                  nullptr, nullptr, nullptr, stream);
    VGPU_HIP(hipGetLastError());
    VGPU_HIP(hipMemcpyAsync(ids, w_ids.p, nq * k * sizeof(int64_t), hipMemcpyDeviceToHost, stream));
    VGPU_HIP(hipMemcpyAsync(dists, w_odist.p, nq * k * sizeof(float), hipMemcpyDeviceToHost, stream));
    VGPU_HIP(hipStreamSynchronize(stream));
}

}  // namespace vgpu
