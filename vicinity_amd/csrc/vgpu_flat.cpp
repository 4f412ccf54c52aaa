// Flat exact index: database resident in HBM, batched top-k.
// Reference: brute force over l2_distance_squared / cosine_distance_normalized
// (src/distance.rs:78-109), as the reference's ground truth
// (src/ivf_pq/search.rs:3376-3392, tests/common/mod.rs:49-57).
#include <algorithm>
#include <cmath>

#include "vgpu_runtime.h"

namespace vgpu {

// Flagged queries the ranking path's fallback takes with the count read on the device
constexpr size_t kFlatFallbackCap = 256;

FlatIndex::FlatIndex(size_t dim, int met) : d(dim), metric(met) {
    if (dim == 0) throw Error(VGPU_ERR_INVALID_CONFIG, "dimension must be greater than 0");
    if (met != 0 && met != 1) throw Error(VGPU_ERR_INVALID_CONFIG, "metric must be 0 (L2) or 1 (1 - dot)");
    VGPU_HIP(hipStreamCreate(&stream));
    for (auto& e : ev) VGPU_HIP(hipEventCreate(&e));
}

FlatIndex::~FlatIndex() {
    if (stream) (void)hipStreamSynchronize(stream);
    for (auto& e : ev)
        if (e) (void)hipEventDestroy(e);
    if (stream) (void)hipStreamDestroy(stream);
}

void FlatIndex::add(const float* x, size_t count) {
    if (n + count >= 0xffffffffull) throw Error(VGPU_ERR_INVALID_PARAMETER, "more than 2^32-1 vectors");
    const size_t n0 = n;
    const double xmax0 = xmax2;
    host.insert(host.end(), x, x + count * d);
    for (size_t i = 0; i < count; i++) {
        double t = 0.0;
        for (size_t j = 0; j < d; j++) t += (double)x[i * d + j] * x[i * d + j];
        xmax2 = std::max(xmax2, t);
    }
    n += count;
    try {
        sync_device();
    } catch (...) {
        // A failed allocation has released the buffer it was growing: go
        // back to the previous rows and rebuild their device copy.
        host.resize(n0 * d);
        n = n0;
        xmax2 = xmax0;
        try {
            sync_device();
        } catch (...) {
            stale = true;
        }
        throw;
    }
}

void FlatIndex::sync_device() {
    stale = true;
    if (n) {
        d_x.upload(host.data(), n * d, stream);
        d_xnorm.reserve(n);
        launch_flat_norms(d_x.p, (int)n, (int)d, d_xnorm.p, stream);
        if (flat_pack_chunks((int)n, (int)d)) {
            d_xb.reserve(flat_pack_chunks((int)n, (int)d));
            launch_flat_pack(d_x.p, (int)n, (int)d, d_xb.p, stream);
        }
        VGPU_HIP(hipGetLastError());
        VGPU_HIP(hipStreamSynchronize(stream));
    }
    stale = false;
}

void FlatIndex::search_device(const float* d_q, size_t nq, size_t k, int64_t* d_ids, float* d_dists,
                              hipStream_t s) {
    if (!s) s = stream;
    if (stale)
        throw Error(VGPU_ERR_DEVICE, "the device copy of the flat index was lost in a failed add; add again");
    if (nq == 0 || k == 0) return;
    if (k > 112) throw Error(VGPU_ERR_INVALID_PARAMETER, "flat search supports k <= 112");
    if (n == 0) {
        launch_finalize(nullptr, nullptr, nullptr, (int)nq, 0, (int)k, d_ids, d_dists, s);
        VGPU_HIP(hipStreamSynchronize(s));
        return;
    }
    const float xmax = (float)(std::sqrt(xmax2) * 1.0001 + 1e-30);
    w_qnorm.reserve(nq);
    w_partial.reserve(flat_partial_count((int)nq, (int)n, (int)d, (int)k));
    w_idx.reserve(nq * k);
    w_dist.reserve(nq * k);
    w_overflow.reserve(1);
    w_flag.reserve(nq);
    w_fb.reserve(nq);
    VGPU_HIP(hipMemsetAsync(w_overflow.p, 0, sizeof(unsigned int), s));
    // the bf16x3 ranking path computes the query norms in its merge
    const int rsl = d_xb.n ? flat_rank_fallback_slices((int)nq, (int)n, (int)d, (int)k) : 0;
    if (!rsl) launch_flat_norms(d_q, (int)nq, (int)d, w_qnorm.p, s);
    VGPU_HIP(hipEventRecord(ev[0], s));
    launch_flat_search(d_q, rsl ? nullptr : w_qnorm.p, (int)nq, d_x.p, d_xb.n ? d_xb.p : nullptr, d_xnorm.p,
                       (int)n, (int)d, (int)k, metric, xmax, w_partial.p, w_idx.p, w_dist.p, w_overflow.p, w_flag.p,
                       w_fb.p, s, ev[3]);
    // the unproved queries (rare): exact scans over many workgroups.  The
    // ranking path runs the first kFlatFallbackCap of them with the count
    // read on the device (no host round trip), the rest after the final
    // wait; the other path reads the count first.
    const int cap = rsl ? (int)std::min<size_t>(nq, kFlatFallbackCap) : 0;
    if (rsl) {
        w_fbkeys.reserve((size_t)cap * rsl * k);
        launch_flat_rank_fallback_dev(w_flag.p, w_overflow.p, cap, w_fb.p, w_partial.p, (int)nq, (int)n, (int)d,
                                      (int)k, metric, d_q, d_x.p, w_fbkeys.p, w_idx.p, w_dist.p, s);
    } else {
        VGPU_HIP(hipMemcpyAsync(&fallbacks, w_overflow.p, sizeof(unsigned int), hipMemcpyDeviceToHost, s));
        VGPU_HIP(hipStreamSynchronize(s));
        if (fallbacks) {
            w_fbkeys.reserve((size_t)fallbacks * flat_fallback_slices((int)n, (int)k) * k);
            launch_flat_fallback(w_flag.p, (int)fallbacks, d_q, d_x.p, (int)n, (int)d, (int)k, metric,
                                 w_fbkeys.p, w_idx.p, w_dist.p, s);
        }
    }
    VGPU_HIP(hipEventRecord(ev[1], s));
    launch_finalize(w_idx.p, w_dist.p, nullptr, (int)nq, (int)k, (int)k, d_ids, d_dists, s);
    VGPU_HIP(hipEventRecord(ev[2], s));
    if (rsl) VGPU_HIP(hipMemcpyAsync(&fallbacks, w_overflow.p, sizeof(unsigned int), hipMemcpyDeviceToHost, s));
    VGPU_HIP(hipGetLastError());
    VGPU_HIP(hipStreamSynchronize(s));
    if (rsl && fallbacks > (unsigned int)cap) {  // more than the device-driven pass took
        const int rest = (int)fallbacks - cap;
        w_fbkeys.reserve((size_t)rest * rsl * k);
        launch_flat_rank_fallback(w_flag.p + cap, rest, w_fb.p, w_partial.p, (int)nq, (int)n, (int)d, (int)k,
                                  metric, d_q, d_x.p, w_fbkeys.p, w_idx.p, w_dist.p, s);
        launch_finalize(w_idx.p, w_dist.p, nullptr, (int)nq, (int)k, (int)k, d_ids, d_dists, s);
        VGPU_HIP(hipEventRecord(ev[2], s));
        VGPU_HIP(hipGetLastError());
        VGPU_HIP(hipStreamSynchronize(s));
    }
    VGPU_HIP(hipEventElapsedTime(&ms_gemm, ev[0], ev[3]));
    VGPU_HIP(hipEventElapsedTime(&ms_total, ev[0], ev[2]));
}

}  // namespace vgpu
