/*
 * vicinity_oracle.h -- CPU restatement of vicinity's IVF-PQ search path.
 *
 * TEST INFRASTRUCTURE ONLY.  Results are checked against this library: it is
 * loaded by tests/, by __graft_entry__.smoke() and by bench.py's cpu_baseline
 * leg, and never by the product (vicinity_amd/).  Every function cites the reference
 * file:line it restates (paths relative to the vicinity repository root).
 *
 * Arithmetic rules (all in IEEE binary32, compiled with -ffp-contract=off and
 * without -ffast-math, so every `a*b + c` rounds twice exactly like Rust):
 *   - dot / squared-L2 are sequential left-to-right sums starting at 0.0
 *     (src/simd.rs:86-121, the scalar backend; the SIMD `innr` backend's
 *     summation order is not published, see the parity notes in the header of
 *     vicinity_oracle.c);
 *   - sums over codebooks run m = 0..M-1 starting at 0.0 (src/pq_simd.rs:349-355);
 *   - top-k ordering is `total_cmp` on the distance; the reference leaves the
 *     order of equal distances unspecified (select_nth_unstable), the oracle
 *     breaks ties by the lower vector (insertion) index.
 */
#ifndef VICINITY_ORACLE_H
#define VICINITY_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- scalar kernels ---------------------------------------------------- */
float or_dot(const float *a, const float *b, size_t n);
float or_l2sq(const float *a, const float *b, size_t n);
void or_normalize(const float *x, size_t d, float *out);
void or_normalize_rows(const float *x, size_t n, size_t d, float *out);

/* ---- product quantiser (src/ivf_pq/pq.rs) ------------------------------ */
void or_adc_table(const float *codebooks, size_t M, size_t K, size_t ds,
                  const float *r, float *table);
float or_distance_with_table(const float *table, size_t M, size_t K,
                             const uint8_t *codes);
void or_adc_scan(const uint8_t *codes, size_t n, size_t M, size_t K,
                 const float *table, float *out);
void or_pq_encode(const float *codebooks, size_t M, size_t K, size_t ds,
                  const float *x, size_t n, uint8_t *codes);
void or_pq_reconstruct(const float *codebooks, size_t M, size_t K, size_t ds,
                       const uint8_t *codes, float *out);

/* ---- FastScan 4-bit (src/pq_simd.rs:400-769) --------------------------- */
size_t or_pack4_size(size_t n, size_t M);
void or_pack4(const uint8_t *codes, size_t n, size_t M, uint8_t *out);
void or_quantize_lut(const float *lut, size_t M, uint8_t *q, float *scale,
                     float *offset);
void or_fastscan_block(const uint8_t *block, const uint8_t *lutq, size_t M,
                       uint16_t acc[32]);
int or_fastscan_batch(const uint8_t *packed, size_t n, size_t M,
                      const float *lut, float *out);

/* ---- coarse quantiser / top-k (src/ivf_pq/search.rs) ------------------- */
size_t or_nearest_centroids(const float *q, const float *centroids, size_t L,
                            size_t d, size_t nprobe, uint32_t *lists,
                            float *scores);
size_t or_top_k(const uint32_t *idx, const float *dist, size_t n, size_t k,
                uint32_t *out_idx, float *out_dist);

/* ---- index artifacts ------------------------------------------------------
 * The arrays an IVFPQIndex holds after build() (search.rs:212-239):
 *   centroids  f32[L*d]          flat, row-major
 *   codebooks  f32[M*K*ds]       codebook-major, then codeword, then dim
 *   list_offsets u64[L+1]        inverted list l = list_ids[off[l]..off[l+1]]
 *   list_ids   u32[n]            insertion indices, ascending inside a list
 *   codes      u8[n*M]           PQ codes in insertion order (quantized_codes)
 *   doc_ids    u32[n]            insertion index -> caller id
 *   vectors    f32[n*d] or NULL  normalised raw vectors (for rerank)
 *   rotation   f32[d*d] or NULL  OPQ rotation R, row-major (opq.rs:37-38);
 *                                NULL = Quantizer::Product                */
typedef struct or_index {
    size_t d, L, M, K, ds, n;
    const float *centroids;
    const float *codebooks;
    const uint64_t *list_offsets;
    const uint32_t *list_ids;
    const uint8_t *codes;
    const uint32_t *doc_ids;
    const float *vectors;
    const float *rotation;
} or_index;

/* Returns the number of results (<= k); negative on error. */
long or_ivfpq_search(const or_index *ix, const float *query, size_t k,
                     size_t nprobe, uint32_t *out_ids, float *out_dists);
long or_ivfpq_search_reranked(const or_index *ix, const float *query, size_t k,
                              size_t pool, size_t nprobe, uint32_t *out_ids,
                              float *out_dists);
/* Batch: (nq, k) rows padded with (-1, +inf); threads <= 0 means all cores. */
int or_ivfpq_search_batch(const or_index *ix, const float *queries, size_t nq,
                          size_t k, size_t nprobe, size_t rerank_pool,
                          int threads, int64_t *out_ids, float *out_dists);
/* search_with_filter with an equality on the filter field: list_mask[L] the
 * build-time category bitmasks, cat[n] the vectors' categories (-1: none).
 * Returns the number of results (<= k), -1 for a category outside 0..63. */
long or_ivfpq_search_filtered(const or_index *ix, const uint64_t *list_mask,
                              const int8_t *cat, const float *query, size_t k,
                              size_t nprobe, int category, uint32_t *out_ids,
                              float *out_dists);
void or_list_masks(const or_index *ix, const int8_t *cat, uint64_t *list_mask);
/* The probed lists of one query in probe order (ascending coarse distance). */
size_t or_ivfpq_probe(const or_index *ix, const float *query, size_t nprobe,
                      uint32_t *lists, float *scores);

/* ---- build side ------------------------------------------------------- */
void or_assign_cosine(const float *x, size_t n, const float *centroids,
                      size_t L, size_t d, uint32_t *assign);
void or_build_lists(const uint32_t *assign, size_t n, size_t L,
                    uint64_t *offsets, uint32_t *ids);
void or_sample_indices(size_t n, size_t sample, uint64_t seed, uint32_t *out);
/* metric 0 = cosine (spherical k-means), 1 = squared L2.  Returns iterations. */
long or_kmeans(const float *x, size_t n, size_t d, size_t k, int metric,
               uint64_t seed, size_t max_iter, float *centroids);
/* use_opq != 0 trains OPQ on the residuals (search.rs:732-749) and writes
 * its rotation to rotation[d*d]; otherwise rotation is not touched. */
int or_ivfpq_build(const float *vectors, size_t n, size_t d, size_t L,
                   size_t M, size_t K, uint64_t seed, size_t sample,
                   size_t max_iter, int use_opq, float *centroids,
                   float *codebooks, uint32_t *assign, uint8_t *codes,
                   float *rotation, size_t *K_actual);

/* ---- OPQ (src/ivf_pq/opq.rs) ------------------------------------------ */
/* out = R v and out = R^T v, R row-major d x d (opq.rs:180-205). */
void or_matvec(const float *R, const float *v, size_t d, float *out);
void or_matvec_t(const float *R, const float *v, size_t d, float *out);
/* The orthogonal factor U V^T of M = U S V^T (opq.rs:280-294), M row-major
 * d x d float32; computed in float64 by one-sided Jacobi and rounded. */
void or_polar(const float *M, size_t d, float *R);
/* OptimizedProductQuantizer::fit (opq.rs:65-109): rotation[d*d] and the
 * codebooks of the last PQ fit; each PQ fit is this project's k-means with
 * seed + m and max_iter.  Returns 0, or -1 when n < K (opq.rs:71-76). */
int or_opq_fit(const float *data, size_t n, size_t d, size_t M, size_t K,
               size_t iterations, uint64_t seed, size_t max_iter,
               float *rotation, float *codebooks, size_t *K_actual);

/* ---- flat exact search (src/distance.rs:78-109) ----------------------- */
int or_flat_search(const float *base, size_t n, size_t d, const float *queries,
                   size_t nq, size_t k, int metric, int threads,
                   int64_t *out_ids, float *out_dists);

#ifdef __cplusplus
}
#endif
#endif
