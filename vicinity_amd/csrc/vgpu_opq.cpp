// OPQ on the GPU path: training (OptimizedProductQuantizer::fit) with the
// rotations, encodes and the Procrustes sum on the GPU and the polar factor on
// the host, and the rotated residuals the search scans with.
//
// Reference: src/ivf_pq/opq.rs fit :65-109, compute_optimal_rotation
// :232-295, quantize :112-115, approximate_distance_table :120-123; the IVF-PQ
// build calls opq.fit(training residuals, count, 10) (search.rs:732-749).
// This file is compiled with -ffp-contract=off.
#include <algorithm>
#include <cmath>
#include <cstring>

#include "vgpu_runtime.h"

namespace vgpu {

// One-sided Jacobi (Hestenes; Demmel & Veselic 1992) in float64: column pairs
// of A = M are rotated until every pair is orthogonal to 1e-15 (at most 64
// sweeps), the rotations accumulated in V, so that A = U S.  Columns of norm
// <= 1e-12 of the largest (M rank-deficient) are completed in column order by
// the unit vector with the largest component outside the columns so far
// (Gram-Schmidt, two passes, lowest index on ties).  R = U V^T, rounded.
// opq.rs:280-294 takes the same factor from nalgebra's SVD.  A, V and U are
// stored transposed (column j is row j), so a column pair is two contiguous
// rows; every sum still runs over k in ascending order.
void polar_factor(const float* Mf, size_t d, float* R) {
    std::vector<double> At(d * d), Vt(d * d, 0.0), Ut(d * d, 0.0), u(d), best(d), nrm(d), S(d * d, 0.0);
    std::vector<char> ok(d, 0);
    for (size_t k = 0; k < d; k++)
        for (size_t j = 0; j < d; j++) At[j * d + k] = (double)Mf[k * d + j];
    for (size_t i = 0; i < d; i++) Vt[i * d + i] = 1.0;
    for (int sweep = 0; sweep < 64; sweep++) {
        bool changed = false;
        for (size_t p = 0; p + 1 < d; p++)
            for (size_t q = p + 1; q < d; q++) {
                double* ap = &At[p * d];
                double* aq = &At[q * d];
                double a = 0.0, b = 0.0, g = 0.0;
                for (size_t k = 0; k < d; k++) {
                    const double x = ap[k], y = aq[k];
                    a += x * x;
                    b += y * y;
                    g += x * y;
                }
                if (g == 0.0 || std::fabs(g) <= 1e-15 * std::sqrt(a * b)) continue;
                const double z = (b - a) / (2.0 * g);
                const double t = (z >= 0.0 ? 1.0 : -1.0) / (std::fabs(z) + std::sqrt(1.0 + z * z));
                const double c = 1.0 / std::sqrt(1.0 + t * t), sn = c * t;
                double* vp = &Vt[p * d];
                double* vq = &Vt[q * d];
                for (size_t k = 0; k < d; k++) {
                    const double x = ap[k], y = aq[k];
                    ap[k] = c * x - sn * y;
                    aq[k] = sn * x + c * y;
                }
                for (size_t k = 0; k < d; k++) {
                    const double x = vp[k], y = vq[k];
                    vp[k] = c * x - sn * y;
                    vq[k] = sn * x + c * y;
                }
                changed = true;
            }
        if (!changed) break;
    }
    double smax = 0.0;
    for (size_t j = 0; j < d; j++) {
        double s2 = 0.0;
        for (size_t k = 0; k < d; k++) s2 += At[j * d + k] * At[j * d + k];
        nrm[j] = std::sqrt(s2);
        if (nrm[j] > smax) smax = nrm[j];
    }
    for (size_t j = 0; j < d; j++)
        if (nrm[j] > 0.0 && nrm[j] > 1e-12 * smax) {
            ok[j] = 1;
            for (size_t k = 0; k < d; k++) Ut[j * d + k] = At[j * d + k] / nrm[j];
        }
    for (size_t j = 0; j < d; j++) {
        if (ok[j]) continue;
        double bn = -1.0;
        for (size_t e = 0; e < d; e++) {
            for (size_t k = 0; k < d; k++) u[k] = k == e ? 1.0 : 0.0;
            for (int pass = 0; pass < 2; pass++)
                for (size_t c = 0; c < d; c++) {
                    if (!ok[c]) continue;
                    const double* uc = &Ut[c * d];
                    double pr = 0.0;
                    for (size_t k = 0; k < d; k++) pr += uc[k] * u[k];
                    for (size_t k = 0; k < d; k++) u[k] -= pr * uc[k];
                }
            double s2 = 0.0;
            for (size_t k = 0; k < d; k++) s2 += u[k] * u[k];
            if (s2 > bn) {
                bn = s2;
                best = u;
            }
        }
        bn = std::sqrt(bn);
        for (size_t k = 0; k < d; k++) Ut[j * d + k] = best[k] / bn;
        ok[j] = 1;
    }
    // R[i][j] = sum over k ascending of U[i][k] V[j][k] = Ut[k][i] Vt[k][j]
    for (size_t k = 0; k < d; k++) {
        const double* uk = &Ut[k * d];
        const double* vk = &Vt[k * d];
        for (size_t i = 0; i < d; i++) {
            const double ui = uk[i];
            double* si = &S[i * d];
            for (size_t j = 0; j < d; j++) si[j] += ui * vk[j];
        }
    }
    for (size_t i = 0; i < d * d; i++) R[i] = (float)S[i];
}

// OptimizedProductQuantizer::fit(res, nt, 10) (opq.rs:65-109): R starts as
// the identity; each iteration trains PQ on the rows rotated by R (the rows as
// given in the first), then sums M += reconstruct(quantize(R x))^T x over the
// first min(nt, 5000) rows and sets R = polar(M).  The codebooks are those of
// the last PQ fit.  The reference's PQ fits inside OPQ are unseeded with 100
// iterations (pq.rs:61-72); here each is the seeded k-means of train_pq.
void IvfpqIndex::train_opq(const std::vector<float>& res, size_t nt, uint64_t seed) {
    if (d > 2048) throw Error(VGPU_ERR_UNSUPPORTED, "OPQ rotation is limited to dimension <= 2048");
    const size_t ns = std::min<size_t>(nt, 5000);
    rotation.assign(d * d, 0.0f);
    for (size_t i = 0; i < d; i++) rotation[i * d + i] = 1.0f;
    DevBuf<float> dres, drot, drx, dcb, dM;
    DevBuf<uint8_t> dcodes;
    dres.upload(res.data(), nt * d, stream);
    drx.reserve(nt * d);
    dM.reserve(d * d);
    dcodes.reserve(ns * M);
    std::vector<float> rotated(res), Mh(d * d);
    for (int it = 0; it < 10; it++) {
        drot.upload(rotation.data(), d * d, stream);
        if (it > 0) {  // opq.rs:82-93
            launch_rotate_rows(drot.p, dres.p, 1, nullptr, nullptr, 0, nt, (int)d, drx.p, stream);
            VGPU_HIP(hipGetLastError());
            VGPU_HIP(hipMemcpyAsync(rotated.data(), drx.p, nt * d * sizeof(float), hipMemcpyDeviceToHost,
                                    stream));
            VGPU_HIP(hipStreamSynchronize(stream));
        }
        train_pq(rotated, nt, params.codebook_size, seed, 100);  // opq.rs:96
        // compute_optimal_rotation (opq.rs:232-295)
        launch_rotate_rows(drot.p, dres.p, 1, nullptr, nullptr, 0, ns, (int)d, drx.p, stream);
        dcb.upload(codebooks.data(), codebooks.size(), stream);
        launch_encode(drx.p, (int)ns, (int)d, nullptr, nullptr, dcb.p, (int)M, (int)K, (int)ds, dcodes.p,
                      stream);
        launch_procrustes(dcodes.p, dcb.p, (int)M, (int)K, (int)ds, dres.p, (int)ns, (int)d, dM.p, stream);
        VGPU_HIP(hipGetLastError());
        VGPU_HIP(hipMemcpyAsync(Mh.data(), dM.p, d * d * sizeof(float), hipMemcpyDeviceToHost, stream));
        VGPU_HIP(hipStreamSynchronize(stream));
        polar_factor(Mh.data(), d, rotation.data());
    }
}

void IvfpqIndex::set_rotation(const float* R) {
    if (built) throw Error(VGPU_ERR_ALREADY_BUILT, "the rotation of a built index is fixed");
    if (!R) {
        rotation.clear();
        return;
    }
    if (!params.use_opq)
        throw Error(VGPU_ERR_INVALID_CONFIG, "a rotation needs an index made with use_opq");
    if (d > 2048) throw Error(VGPU_ERR_UNSUPPORTED, "OPQ rotation is limited to dimension <= 2048");
    for (size_t i = 0; i < d * d; i++)
        if (!std::isfinite(R[i])) throw Error(VGPU_ERR_INVALID_PARAMETER, "rotation contains a non-finite value");
    rotation.assign(R, R + d * d);
}

// R (q_i - c_l) for every slot (i, p), l = d_lists[i * P + p] (slots >= L
// give zero rows, never scanned), into out[nq * P * d].
void IvfpqIndex::rotate_slots(const float* d_qn, size_t nq, size_t P, const uint32_t* d_lists, float* out,
                              hipStream_t s) {
    launch_rotate_rows(d_rotation.p, d_qn, (int)P, d_centroids.p, d_lists, (int)L, nq * P, (int)d, out, s);
    VGPU_HIP(hipGetLastError());
}

}  // namespace vgpu
