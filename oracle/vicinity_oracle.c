/*
 * vicinity_oracle.c -- CPU restatement of vicinity's IVF-PQ search path.
 *
 * TEST INFRASTRUCTURE ONLY (results are checked against it; it is never the
 * product).  Loaded by tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg.
 *
 * Reference files (vicinity repository root):
 *   src/ivf_pq/search.rs   normalize_query 55-62, finish_top_k_by_distance 64-75,
 *                          add_slice 488-512, build 546-787, training_indices
 *                          789-814, build_scan_caches 816-848, search 1087-1093,
 *                          search_reranked 1117-1158, search_approx_internal_observed
 *                          1175-1391, search_with_filter 1407-1549,
 *                          find_nearest_centroids 1602-1617
 *   src/ivf_pq/opq.rs      fit 65-109, quantize 112-115, approximate_distance_table
 *                          120-123, matrix products 180-205, compute_optimal_rotation
 *                          232-295
 *   src/ivf_pq/pq.rs       fit 75-124, quantize 136-161, compute_adc_table_into
 *                          196-266, distance_with_table 272-279, reconstruct 284-290
 *   src/pq_simd.rs         adc_batch_distances_into 99-115, adc_batch_256_into
 *                          330-369, PackedCodes4bit::pack 426-486,
 *                          FASTSCAN_MAX_CODEBOOKS 517, quantize_lut_flat 576-611,
 *                          fastscan_block_portable 629-654,
 *                          fastscan_batch_quantized 721-769
 *   src/distance.rs        l2_distance_squared 78-83, cosine_distance_normalized 104-109
 *   src/simd.rs            scalar backend dot 86-91, l2_distance_squared 118-121
 *   src/python.rs          batch_search padding 744-793, MISSING_LABEL 1303-1304
 *
 * Parity status of each function (how it is pinned; tests/test_oracle_*.py):
 *   or_dot / or_l2sq / or_normalize        closed forms (simd.rs:129-160 values,
 *                                          3-4-5), brute force in float64
 *   or_adc_table                           KATs pq.rs:335-372, float64 identity
 *                                          sum == ||q - reconstruct||^2 (pq.rs:435-478)
 *   or_adc_scan / or_distance_with_table   bitwise vs m-ordered naive sum
 *                                          (pq_simd.rs:1108-1132), KAT 154.2
 *   or_pack4 / or_quantize_lut /
 *   or_fastscan_*                          layout KAT pq_simd.rs:1041-1077, u16
 *                                          limit 780-795, range KAT 1160-1187,
 *                                          error bound 1206-1318
 *   or_top_k                               KAT search.rs:2047-2069, brute sort
 *   or_flat_search                         closed forms (distance.rs:78-83,
 *                                          104-109 values), metric branches that
 *                                          rank in opposite orders, ties by index,
 *                                          k > n padding, float64 brute force,
 *                                          each distance = its pair's primitive
 *   or_nearest_centroids                   brute force sort of float64 scores
 *   or_ivfpq_search                        full probe == exhaustive ADC scan
 *                                          over reconstruct (search.rs:2589-2645)
 *   or_ivfpq_search_filtered / or_list_masks  the widening case of
 *                                          search.rs:2652-2688 (the three tagged
 *                                          documents behind nprobe = 1), full
 *                                          probe == exhaustive scan of the
 *                                          category over reconstruct, results
 *                                          carry the category
 *   or_pq_encode                           argmin property (pq.rs:485-551)
 *   or_assign_cosine                       float64 argmin of 1 - x.c wherever the
 *                                          float32 rounding bound separates it,
 *                                          equals or_nearest_centroids(.., 1),
 *                                          exact ties (duplicated centroids, zero
 *                                          row, d = 1) go to the lowest index
 *   or_matvec / or_matvec_t                KATs opq.rs:362-385, float64 products,
 *                                          a permutation exactly
 *   or_polar                               numpy (LAPACK) SVD U V^T, R^T M
 *                                          symmetric PSD, M = Q D gives Q; the
 *                                          reference's nalgebra 0.35 float32 SVD
 *                                          (absent) is unpinned to the last bit
 *   or_opq_fit                             the reference's OPQ tests
 *                                          (opq.rs:309-453, tests/opq_vs_pq.rs
 *                                          MAE bounds), the last rotation is
 *                                          polar of the last fit; its PQ fits are
 *                                          seeded here, unseeded in the reference
 *   or_kmeans / or_ivfpq_build             the reference trains with the `clump`
 *                                          crate (^0.7.0, absent): this k-means
 *                                          is this project's own definition and
 *                                          is pinned only by invariants
 *                                          (assignments are argmins, centroids
 *                                          are member means) -- parity with
 *                                          clump's centroids is unpinned.
 * The reference's default SIMD backend (`innr` ^0.7.3, absent) publishes no
 * summation order: at near-ties the oracle follows the scalar backend of
 * src/simd.rs, which is the reference's own build without `innr`.
 */
#include "vicinity_oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>
#include <unistd.h>

#define OR_SIMD_BATCH_THRESHOLD 16   /* search.rs:30-32 */
#define OR_FASTSCAN_MAX_CODEBOOKS 257 /* pq_simd.rs:517 (65535 / 255) */

/* ------------------------------------------------------------------------ */
/* scalar kernels                                                           */
/* ------------------------------------------------------------------------ */

/* simd.rs:88-91 (scalar backend): sequential sum of products from 0.0. */
float or_dot(const float *a, const float *b, size_t n) {
    float s = 0.0f;
    for (size_t i = 0; i < n; i++) s += a[i] * b[i];
    return s;
}

/* simd.rs:118-121: sum of (x - y)^2, sequential; powi(2) is one multiply. */
float or_l2sq(const float *a, const float *b, size_t n) {
    float s = 0.0f;
    for (size_t i = 0; i < n; i++) {
        float t = a[i] - b[i];
        s += t * t;
    }
    return s;
}

/* search.rs:55-62 (query) and :503-508 (insert): x / ||x|| if ||x|| > 1e-10. */
void or_normalize(const float *x, size_t d, float *out) {
    float s = 0.0f;
    for (size_t i = 0; i < d; i++) s += x[i] * x[i];
    float norm = sqrtf(s);
    if (norm > 1e-10f) {
        for (size_t i = 0; i < d; i++) out[i] = x[i] / norm;
    } else if (out != x) {
        memcpy(out, x, d * sizeof(float));
    }
}

void or_normalize_rows(const float *x, size_t n, size_t d, float *out) {
    for (size_t i = 0; i < n; i++) or_normalize(x + i * d, d, out + i * d);
}

/* f32::total_cmp as an unsigned key: negative values flip all bits, the rest
 * get the sign bit set, so u32 order == total_cmp order (NaN sorts last). */
static inline uint32_t fkey(float f) {
    uint32_t b;
    memcpy(&b, &f, 4);
    return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}

static inline uint64_t cand_key(float dist, uint32_t idx) {
    return ((uint64_t)fkey(dist) << 32) | idx;
}

/* ------------------------------------------------------------------------ */
/* product quantiser                                                        */
/* ------------------------------------------------------------------------ */

/* pq.rs:196-266.  Table layout [m][k], m-major. */
void or_adc_table(const float *cb, size_t M, size_t K, size_t ds,
                  const float *r, float *table) {
    if (ds == 1) {
        /* pq.rs:211-228: one-dimensional subvectors, out = diff * diff. */
        for (size_t m = 0; m < M; m++) {
            for (size_t k = 0; k < K; k++) {
                float diff = r[m] - cb[m * K + k];
                table[m * K + k] = diff * diff;
            }
        }
        return;
    }
    if (ds <= 8) {
        /* pq.rs:232-251: dist = 0; for dim: diff = q - c; dist += diff*diff. */
        for (size_t m = 0; m < M; m++) {
            const float *qs = r + m * ds;
            for (size_t k = 0; k < K; k++) {
                const float *cw = cb + (m * K + k) * ds;
                float dist = 0.0f;
                for (size_t j = 0; j < ds; j++) {
                    float diff = qs[j] - cw[j];
                    dist += diff * diff;
                }
                table[m * K + k] = dist;
            }
        }
        return;
    }
    /* pq.rs:253-263: l2_distance_squared per codeword (scalar backend). */
    for (size_t m = 0; m < M; m++)
        for (size_t k = 0; k < K; k++)
            table[m * K + k] = or_l2sq(r + m * ds, cb + (m * K + k) * ds, ds);
}

/* pq.rs:272-279: m-ordered sum from 0.0. */
float or_distance_with_table(const float *table, size_t M, size_t K,
                             const uint8_t *codes) {
    float s = 0.0f;
    for (size_t m = 0; m < M; m++) s += table[m * K + codes[m]];
    return s;
}

/* pq_simd.rs:330-369 (K = 256, four candidates interleaved, each still summed
 * m = 0..M-1 from 0.0) and :99-115 (other K): both equal the m-ordered sum. */
void or_adc_scan(const uint8_t *codes, size_t n, size_t M, size_t K,
                 const float *table, float *out) {
    for (size_t i = 0; i < n; i++)
        out[i] = or_distance_with_table(table, M, K, codes + i * M);
}

/* pq.rs:136-161: per subspace, argmin over codewords of the squared L2
 * distance, strict `<` so the lowest code wins ties. */
void or_pq_encode(const float *cb, size_t M, size_t K, size_t ds,
                  const float *x, size_t n, uint8_t *codes) {
    size_t d = M * ds;
    for (size_t i = 0; i < n; i++) {
        for (size_t m = 0; m < M; m++) {
            const float *sub = x + i * d + m * ds;
            uint8_t best = 0;
            float best_dist = INFINITY;
            for (size_t k = 0; k < K; k++) {
                float dist = or_l2sq(sub, cb + (m * K + k) * ds, ds);
                if (dist < best_dist) {
                    best_dist = dist;
                    best = (uint8_t)(k < 255 ? k : 255);
                }
            }
            codes[i * M + m] = best;
        }
    }
}

/* pq.rs:284-290: concatenate codewords. */
void or_pq_reconstruct(const float *cb, size_t M, size_t K, size_t ds,
                       const uint8_t *codes, float *out) {
    for (size_t m = 0; m < M; m++)
        memcpy(out + m * ds, cb + (m * K + codes[m]) * ds, ds * sizeof(float));
}

/* ------------------------------------------------------------------------ */
/* FastScan 4-bit                                                           */
/* ------------------------------------------------------------------------ */

size_t or_pack4_size(size_t n, size_t M) { return ((n + 31) / 32) * 16 * M; }

/* pq_simd.rs:426-486: 32-vector blocks; per codebook 16 bytes; byte[lane] =
 * low nibble of vector lane | low nibble of vector lane+16 << 4; zero pad. */
void or_pack4(const uint8_t *codes, size_t n, size_t M, uint8_t *out) {
    size_t nb = (n + 31) / 32, bpb = 16 * M;
    memset(out, 0, nb * bpb);
    for (size_t b = 0; b < nb; b++) {
        size_t base = b * 32;
        for (size_t m = 0; m < M; m++) {
            for (size_t lane = 0; lane < 16; lane++) {
                size_t lo = base + lane, hi = base + 16 + lane;
                uint8_t clo = lo < n ? (codes[lo * M + m] & 0x0F) : 0;
                uint8_t chi = hi < n ? (codes[hi * M + m] & 0x0F) : 0;
                out[b * bpb + m * 16 + lane] = (uint8_t)(clo | (chi << 4));
            }
        }
    }
}

/* Rust `f32::round().clamp(0.0, 255.0) as u8`: half away from zero; the
 * float->u8 cast saturates and maps NaN to 0. */
static inline uint8_t round_to_u8(float v) {
    float r = roundf(v);
    if (!(r >= 0.0f)) return 0; /* negative or NaN */
    if (r > 255.0f) return 255;
    return (uint8_t)r;
}

/* pq_simd.rs:576-611. */
void or_quantize_lut(const float *lut, size_t M, uint8_t *q, float *scale,
                     float *offset) {
    size_t n = M * 16;
    if (n == 0) {
        *scale = 1.0f;
        *offset = 0.0f;
        return;
    }
    float gmin = INFINITY, gmax = -INFINITY;
    for (size_t i = 0; i < n; i++) {
        float v = lut[i];
        if (v < gmin) gmin = v;
        if (v > gmax) gmax = v;
    }
    float range = gmax - gmin;
    float sc, inv;
    if (range < 1.1920929e-07f) { /* f32::EPSILON */
        sc = 1.0f;
        inv = 0.0f;
    } else {
        sc = range / 255.0f;
        inv = 255.0f / range;
    }
    for (size_t i = 0; i < n; i++) q[i] = round_to_u8((lut[i] - gmin) * inv);
    *scale = sc;
    *offset = gmin;
}

/* pq_simd.rs:629-654: u16 accumulation of byte-LUT entries. */
void or_fastscan_block(const uint8_t *block, const uint8_t *lutq, size_t M,
                       uint16_t acc[32]) {
    memset(acc, 0, 32 * sizeof(uint16_t));
    for (size_t m = 0; m < M; m++) {
        for (size_t lane = 0; lane < 16; lane++) {
            uint8_t byte = block[m * 16 + lane];
            acc[lane] = (uint16_t)(acc[lane] + lutq[m * 16 + (byte & 0x0F)]);
            acc[lane + 16] = (uint16_t)(acc[lane + 16] + lutq[m * 16 + (byte >> 4)]);
        }
    }
}

/* pq_simd.rs:716-769: quantise the float LUT, scan every block, convert with
 * `acc as f32 * scale + offset * M` (two roundings, no FMA).
 * Returns -1 when M exceeds the u16 budget (the reference panics). */
int or_fastscan_batch(const uint8_t *packed, size_t n, size_t M,
                      const float *lut, float *out) {
    if (M > OR_FASTSCAN_MAX_CODEBOOKS) return -1;
    uint8_t *lutq = (uint8_t *)malloc(M * 16 + 1);
    float scale, offset;
    or_quantize_lut(lut, M, lutq, &scale, &offset);
    float base_offset = offset * (float)M;
    size_t nb = (n + 31) / 32, bpb = 16 * M;
    uint16_t acc[32];
    for (size_t b = 0; b < nb; b++) {
        or_fastscan_block(packed + b * bpb, lutq, M, acc);
        size_t cnt = n - b * 32;
        if (cnt > 32) cnt = 32;
        for (size_t i = 0; i < cnt; i++) out[b * 32 + i] = (float)acc[i] * scale + base_offset;
    }
    free(lutq);
    return 0;
}

/* ------------------------------------------------------------------------ */
/* selection                                                                */
/* ------------------------------------------------------------------------ */

static int cmp_u64(const void *a, const void *b) {
    uint64_t x = *(const uint64_t *)a, y = *(const uint64_t *)b;
    return x < y ? -1 : (x > y);
}

/* Quickselect (Hoare partition, median-of-three pivot): afterwards
 * keys[0..k) hold the k smallest keys in some order.  Requires 0 < k < n. */
static void select_smallest(uint64_t *a, size_t n, size_t k) {
    size_t lo = 0, hi = n - 1, target = k - 1; /* inclusive range */
    while (lo < hi) {
        if (hi - lo < 16) {
            qsort(a + lo, hi - lo + 1, sizeof(uint64_t), cmp_u64);
            return;
        }
        size_t mid = lo + (hi - lo) / 2;
        uint64_t x = a[lo], y = a[mid], z = a[hi];
        uint64_t pivot = x < y ? (y < z ? y : (x < z ? z : x)) : (x < z ? x : (y < z ? z : y));
        size_t i = lo, j = hi;
        while (i <= j) {
            while (a[i] < pivot) i++;
            while (a[j] > pivot) j--;
            if (i <= j) {
                uint64_t t = a[i];
                a[i] = a[j];
                a[j] = t;
                i++;
                if (j == 0) break;
                j--;
            }
        }
        /* a[lo..j] <= pivot <= a[i..hi]; entries strictly between equal pivot */
        if (target <= j && j != (size_t)-1) hi = j;
        else if (target >= i) lo = i;
        else return;
    }
}

/* search.rs:64-75: the k smallest by total_cmp, ascending; equal distances
 * ordered by index.  Returns min(k, n). */
static size_t top_k_keys(uint64_t *keys, size_t n, size_t k) {
    if (k == 0 || n == 0) return 0;
    if (n > k) select_smallest(keys, n, k);
    size_t m = n < k ? n : k;
    qsort(keys, m, sizeof(uint64_t), cmp_u64);
    return m;
}

size_t or_top_k(const uint32_t *idx, const float *dist, size_t n, size_t k,
                uint32_t *out_idx, float *out_dist) {
    uint64_t *keys = (uint64_t *)malloc((n ? n : 1) * sizeof(uint64_t));
    for (size_t i = 0; i < n; i++) keys[i] = cand_key(dist[i], idx[i]);
    size_t m = top_k_keys(keys, n, k);
    /* recover the distances: find each selected (idx) in the input */
    for (size_t i = 0; i < m; i++) {
        uint32_t id = (uint32_t)keys[i];
        uint32_t kb = (uint32_t)(keys[i] >> 32);
        uint32_t b = (kb & 0x80000000u) ? (kb & 0x7FFFFFFFu) : ~kb;
        float f;
        memcpy(&f, &b, 4);
        out_idx[i] = id;
        out_dist[i] = f;
    }
    free(keys);
    return m;
}

static inline float key_dist(uint64_t key) {
    uint32_t kb = (uint32_t)(key >> 32);
    uint32_t b = (kb & 0x80000000u) ? (kb & 0x7FFFFFFFu) : ~kb;
    float f;
    memcpy(&f, &b, 4);
    return f;
}

/* search.rs:1602-1617: score every centroid with 1 - dot(q, c)
 * (distance.rs:104-109), keep the nprobe smallest, ascending. */
size_t or_nearest_centroids(const float *q, const float *centroids, size_t L,
                            size_t d, size_t nprobe, uint32_t *lists,
                            float *scores) {
    uint64_t *keys = (uint64_t *)malloc((L ? L : 1) * sizeof(uint64_t));
    for (size_t c = 0; c < L; c++)
        keys[c] = cand_key(1.0f - or_dot(q, centroids + c * d, d), (uint32_t)c);
    size_t p = nprobe < L ? nprobe : L;
    size_t m = top_k_keys(keys, L, p);
    for (size_t i = 0; i < m; i++) {
        lists[i] = (uint32_t)keys[i];
        if (scores) scores[i] = key_dist(keys[i]);
    }
    free(keys);
    return m;
}

/* ------------------------------------------------------------------------ */
/* IVF-PQ search                                                            */
/* ------------------------------------------------------------------------ */

size_t or_ivfpq_probe(const or_index *ix, const float *query, size_t nprobe,
                      uint32_t *lists, float *scores) {
    float *qn = (float *)malloc(ix->d * sizeof(float));
    or_normalize(query, ix->d, qn);
    size_t p = or_nearest_centroids(qn, ix->centroids, ix->L, ix->d, nprobe, lists, scores);
    free(qn);
    return p;
}

/* Quantizer::compute_adc_table_into (search.rs:170-181): OPQ rotates the
 * residual first (opq.rs:120-123, rotate_vector :143-148). */
static const float *rotated(const or_index *ix, const float *res, float *rres) {
    if (!ix->rotation) return res;
    or_matvec(ix->rotation, res, ix->d, rres);
    return rres;
}

/* search.rs:1175-1391 up to the candidate list; returns candidate keys
 * (distance, vector index) in *out_keys (malloc'd), count in return. */
static size_t ivfpq_candidates(const or_index *ix, const float *query,
                               size_t nprobe, uint64_t **out_keys) {
    size_t d = ix->d, M = ix->M, K = ix->K, ds = ix->ds;
    float *qn = (float *)malloc(d * sizeof(float));
    float *res = (float *)malloc(d * sizeof(float));
    float *rres = (float *)malloc(d * sizeof(float));
    float *table = (float *)malloc(M * K * sizeof(float));
    or_normalize(query, d, qn); /* :1203 */
    size_t P = nprobe < ix->L ? nprobe : ix->L;
    uint32_t *lists = (uint32_t *)malloc((P ? P : 1) * sizeof(uint32_t));
    P = or_nearest_centroids(qn, ix->centroids, ix->L, d, P, lists, NULL); /* :1213 */
    size_t total = 0;
    for (size_t p = 0; p < P; p++)
        total += (size_t)(ix->list_offsets[lists[p] + 1] - ix->list_offsets[lists[p]]);
    uint64_t *keys = (uint64_t *)malloc((total ? total : 1) * sizeof(uint64_t));
    size_t maxlen = 0;
    for (size_t p = 0; p < P; p++) {
        size_t len = (size_t)(ix->list_offsets[lists[p] + 1] - ix->list_offsets[lists[p]]);
        if (len > maxlen) maxlen = len;
    }
    uint8_t *batch = (uint8_t *)malloc((maxlen ? maxlen : 1) * M);
    uint8_t *packed = (uint8_t *)malloc(or_pack4_size(maxlen ? maxlen : 1, M));
    float *dists = (float *)malloc((maxlen ? maxlen : 1) * sizeof(float));
    size_t nc = 0;
    for (size_t p = 0; p < P; p++) {
        uint32_t l = lists[p];
        const float *c = ix->centroids + (size_t)l * d;
        for (size_t i = 0; i < d; i++) res[i] = qn[i] - c[i]; /* :1242-1245 */
        or_adc_table(ix->codebooks, M, K, ds, rotated(ix, res, rres), table); /* :1255 */
        uint64_t beg = ix->list_offsets[l], end = ix->list_offsets[l + 1];
        size_t len = (size_t)(end - beg);
        const uint32_t *ids = ix->list_ids + beg;
        if (len >= OR_SIMD_BATCH_THRESHOLD) { /* :1261 */
            for (size_t i = 0; i < len; i++)  /* list-major cache, :827-846 */
                memcpy(batch + i * M, ix->codes + (size_t)ids[i] * M, M);
            if (K == 16) { /* FastScan, :1269-1287 */
                or_pack4(batch, len, M, packed);
                or_fastscan_batch(packed, len, M, table, dists);
            } else { /* standard ADC batch, :1318-1344 */
                or_adc_scan(batch, len, M, K, table, dists);
            }
            for (size_t i = 0; i < len; i++) keys[nc++] = cand_key(dists[i], ids[i]);
        } else { /* scalar fallback, :1355-1375 */
            for (size_t i = 0; i < len; i++) {
                float dist = or_distance_with_table(table, M, K, ix->codes + (size_t)ids[i] * M);
                keys[nc++] = cand_key(dist, ids[i]);
            }
        }
    }
    free(qn);
    free(res);
    free(rres);
    free(table);
    free(lists);
    free(batch);
    free(packed);
    free(dists);
    *out_keys = keys;
    return nc;
}

/* search.rs:1087-1093 + :1384: top-k, then vector index -> doc id. */
long or_ivfpq_search(const or_index *ix, const float *query, size_t k,
                     size_t nprobe, uint32_t *out_ids, float *out_dists) {
    uint64_t *keys;
    size_t nc = ivfpq_candidates(ix, query, nprobe, &keys);
    size_t m = top_k_keys(keys, nc, k);
    for (size_t i = 0; i < m; i++) {
        uint32_t vidx = (uint32_t)keys[i];
        out_ids[i] = ix->doc_ids ? ix->doc_ids[vidx] : vidx;
        out_dists[i] = key_dist(keys[i]);
    }
    free(keys);
    return (long)m;
}

/* search.rs:1117-1158: approximate top-max(pool, k), then exact
 * 1 - dot(q_normalised, stored normalised vector), then top-k. */
long or_ivfpq_search_reranked(const or_index *ix, const float *query, size_t k,
                              size_t pool, size_t nprobe, uint32_t *out_ids,
                              float *out_dists) {
    if (!ix->vectors) return -1; /* Unsupported after compact(), :1137-1142 */
    if (pool < k) pool = k;      /* :1144 */
    uint64_t *keys;
    size_t nc = ivfpq_candidates(ix, query, nprobe, &keys);
    size_t m = top_k_keys(keys, nc, pool);
    float *qn = (float *)malloc(ix->d * sizeof(float));
    or_normalize(query, ix->d, qn); /* :1146 */
    for (size_t i = 0; i < m; i++) {
        uint32_t vidx = (uint32_t)keys[i];
        float exact = 1.0f - or_dot(qn, ix->vectors + (size_t)vidx * ix->d, ix->d);
        keys[i] = cand_key(exact, vidx);
    }
    size_t r = top_k_keys(keys, m, k); /* :1157 */
    for (size_t i = 0; i < r; i++) {
        uint32_t vidx = (uint32_t)keys[i];
        out_ids[i] = ix->doc_ids ? ix->doc_ids[vidx] : vidx;
        out_dists[i] = key_dist(keys[i]);
    }
    free(qn);
    free(keys);
    return (long)r;
}

/* search.rs:1407-1549 (search_with_filter, MetadataFilter::Equals on the
 * filter field): list_mask[L] holds each list's build-time category bitmask
 * (search.rs:626-648), cat[n] each vector's current category (-1: none).  The
 * nprobe nearest lists are visited in probe order, lists without the category
 * bit skipped; each visited list's table (pq.rs:196-266) scores its members of
 * the category with distance_with_table (pq.rs:272-279, for every ksub: this
 * path never takes FastScan).  Fewer than k matches with lists left unvisited:
 * every list is visited in index order, the visited ones skipped
 * (:1540-1545).  Then top-k (:1548, :64-75). */
long or_ivfpq_search_filtered(const or_index *ix, const uint64_t *list_mask,
                              const int8_t *cat, const float *query, size_t k,
                              size_t nprobe, int category, uint32_t *out_ids,
                              float *out_dists) {
    if (category < 0 || category > 63) return -1; /* :1435-1450 */
    size_t d = ix->d, M = ix->M, K = ix->K, ds = ix->ds, L = ix->L;
    const uint64_t bit = 1ull << category;
    float *qn = (float *)malloc(d * sizeof(float));
    float *res = (float *)malloc(d * sizeof(float));
    float *rres = (float *)malloc(d * sizeof(float));
    float *table = (float *)malloc(M * K * sizeof(float));
    uint32_t *order = (uint32_t *)malloc((L ? L : 1) * sizeof(uint32_t));
    char *scanned = (char *)calloc(L ? L : 1, 1);
    uint64_t *keys = (uint64_t *)malloc((ix->n ? ix->n : 1) * sizeof(uint64_t));
    or_normalize(query, d, qn); /* :1462-1468 */
    size_t P = nprobe < L ? nprobe : L;
    size_t no = or_nearest_centroids(qn, ix->centroids, L, d, P, order, NULL); /* :1471 */
    size_t nc = 0;
    for (;;) {
        for (size_t o = 0; o < no; o++) {
            uint32_t l = order[o];
            if (scanned[l]) continue;
            scanned[l] = 1;
            if ((list_mask[l] & bit) == 0) continue; /* :1504-1506 */
            const float *c = ix->centroids + (size_t)l * d;
            for (size_t i = 0; i < d; i++) res[i] = qn[i] - c[i]; /* :1509-1512 */
            or_adc_table(ix->codebooks, M, K, ds, rotated(ix, res, rres), table); /* :1514 */
            for (uint64_t p = ix->list_offsets[l]; p < ix->list_offsets[l + 1]; p++) {
                uint32_t v = ix->list_ids[p];
                if (cat[v] != category) continue; /* metadata_store.matches, :1521 */
                float dist = or_distance_with_table(table, M, K, ix->codes + (size_t)v * M);
                keys[nc++] = cand_key(dist, v);
            }
        }
        if (nc >= k || no == L) break; /* :1540 */
        for (size_t l = 0; l < L; l++) order[l] = (uint32_t)l; /* :1545 */
        no = L;
    }
    size_t m = top_k_keys(keys, nc, k);
    for (size_t i = 0; i < m; i++) {
        uint32_t vidx = (uint32_t)keys[i];
        out_ids[i] = ix->doc_ids ? ix->doc_ids[vidx] : vidx;
        out_dists[i] = key_dist(keys[i]);
    }
    free(qn);
    free(res);
    free(rres);
    free(table);
    free(order);
    free(scanned);
    free(keys);
    return (long)m;
}

/* search.rs:626-648: a list's bitmask is the OR of 1 << category over its
 * members that carry a category. */
void or_list_masks(const or_index *ix, const int8_t *cat, uint64_t *list_mask) {
    for (size_t l = 0; l < ix->L; l++) {
        uint64_t msk = 0;
        for (uint64_t p = ix->list_offsets[l]; p < ix->list_offsets[l + 1]; p++) {
            int c = cat[ix->list_ids[p]];
            if (c >= 0 && c < 64) msk |= 1ull << c;
        }
        list_mask[l] = msk;
    }
}

/* ---- batch: python.rs:744-793 (pad with -1 / +inf), run on a thread pool
 * over queries (the rayon par_iter shape of src/hnsw/graph.rs:2716-2727). */
typedef struct {
    const or_index *ix;
    const float *queries;
    size_t nq, k, nprobe, pool;
    int64_t *out_ids;
    float *out_dists;
    size_t next; /* atomic work counter */
    int err;
} batch_job;

static void *batch_worker(void *arg) {
    batch_job *job = (batch_job *)arg;
    size_t k = job->k;
    uint32_t *ids = (uint32_t *)malloc((k ? k : 1) * sizeof(uint32_t));
    float *dists = (float *)malloc((k ? k : 1) * sizeof(float));
    for (;;) {
        size_t i = __atomic_fetch_add(&job->next, 1, __ATOMIC_RELAXED);
        if (i >= job->nq) break;
        const float *q = job->queries + i * job->ix->d;
        long m = job->pool ? or_ivfpq_search_reranked(job->ix, q, k, job->pool, job->nprobe, ids, dists)
                           : or_ivfpq_search(job->ix, q, k, job->nprobe, ids, dists);
        if (m < 0) {
            job->err = 1;
            m = 0;
        }
        for (size_t j = 0; j < k; j++) {
            job->out_ids[i * k + j] = j < (size_t)m ? (int64_t)ids[j] : -1;
            job->out_dists[i * k + j] = j < (size_t)m ? dists[j] : INFINITY;
        }
    }
    free(ids);
    free(dists);
    return NULL;
}

static int resolve_threads(int threads) {
    if (threads > 0) return threads;
    long n = sysconf(_SC_NPROCESSORS_ONLN);
    return n > 0 ? (int)n : 1;
}

int or_ivfpq_search_batch(const or_index *ix, const float *queries, size_t nq,
                          size_t k, size_t nprobe, size_t rerank_pool,
                          int threads, int64_t *out_ids, float *out_dists) {
    batch_job job = {ix, queries, nq, k, nprobe, rerank_pool, out_ids, out_dists, 0, 0};
    int t = resolve_threads(threads);
    if ((size_t)t > nq) t = nq ? (int)nq : 1;
    pthread_t *tids = (pthread_t *)malloc((size_t)t * sizeof(pthread_t));
    for (int i = 0; i < t; i++) pthread_create(&tids[i], NULL, batch_worker, &job);
    for (int i = 0; i < t; i++) pthread_join(tids[i], NULL);
    free(tids);
    return job.err ? -1 : 0;
}

/* ------------------------------------------------------------------------ */
/* build side                                                               */
/* ------------------------------------------------------------------------ */

/* Assignment used by the list build (search.rs:621 -> kmeans.rs:97-107):
 * argmin over centroids of 1 - dot(x, c), strict `<`, lowest index wins. */
void or_assign_cosine(const float *x, size_t n, const float *centroids,
                      size_t L, size_t d, uint32_t *assign) {
    for (size_t i = 0; i < n; i++) {
        uint32_t best = 0;
        float best_s = INFINITY;
        for (size_t c = 0; c < L; c++) {
            float s = 1.0f - or_dot(x + i * d, centroids + c * d, d);
            if (s < best_s) {
                best_s = s;
                best = (uint32_t)c;
            }
        }
        assign[i] = best;
    }
}

static void assign_l2(const float *x, size_t n, const float *centroids,
                      size_t L, size_t d, uint32_t *assign) {
    for (size_t i = 0; i < n; i++) {
        uint32_t best = 0;
        float best_s = INFINITY;
        for (size_t c = 0; c < L; c++) {
            float s = or_l2sq(x + i * d, centroids + c * d, d);
            if (s < best_s) {
                best_s = s;
                best = (uint32_t)c;
            }
        }
        assign[i] = best;
    }
}

/* search.rs:624-657: list l holds the insertion indices assigned to it, in
 * ascending order (counting sort keeps insertion order). */
void or_build_lists(const uint32_t *assign, size_t n, size_t L,
                    uint64_t *offsets, uint32_t *ids) {
    memset(offsets, 0, (L + 1) * sizeof(uint64_t));
    for (size_t i = 0; i < n; i++) offsets[assign[i] + 1]++;
    for (size_t l = 0; l < L; l++) offsets[l + 1] += offsets[l];
    uint64_t *fill = (uint64_t *)malloc((L ? L : 1) * sizeof(uint64_t));
    memcpy(fill, offsets, L * sizeof(uint64_t));
    for (size_t i = 0; i < n; i++) ids[fill[assign[i]]++] = (uint32_t)i;
    free(fill);
}

/* splitmix64 (Steele, Lea, Flood 2014): the seeded stream of this project's
 * training sample and k-means initialisation. */
static inline uint64_t splitmix64(uint64_t *s) {
    uint64_t z = (*s += 0x9E3779B97F4A7C15ull);
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

static inline size_t bounded(uint64_t *s, size_t n) {
    return (size_t)(((unsigned __int128)splitmix64(s) * (unsigned __int128)n) >> 64);
}

/* Partial Fisher-Yates: the first `count` entries of a seeded shuffle of
 * 0..n-1, in draw order. */
static void draw_distinct(size_t n, size_t count, uint64_t seed, uint32_t *out) {
    uint32_t *perm = (uint32_t *)malloc((n ? n : 1) * sizeof(uint32_t));
    for (size_t i = 0; i < n; i++) perm[i] = (uint32_t)i;
    uint64_t s = seed;
    for (size_t i = 0; i < count; i++) {
        size_t j = i + bounded(&s, n - i);
        uint32_t t = perm[i];
        perm[i] = perm[j];
        perm[j] = t;
        out[i] = perm[i];
    }
    free(perm);
}

static int cmp_u32(const void *a, const void *b) {
    uint32_t x = *(const uint32_t *)a, y = *(const uint32_t *)b;
    return x < y ? -1 : (x > y);
}

/* Training sample (the role of search.rs:789-814): sample == 0 or >= n means
 * every vector; otherwise `sample` distinct indices, ascending. */
void or_sample_indices(size_t n, size_t sample, uint64_t seed, uint32_t *out) {
    if (sample == 0 || sample >= n) {
        for (size_t i = 0; i < n; i++) out[i] = (uint32_t)i;
        return;
    }
    draw_distinct(n, sample, seed, out);
    qsort(out, sample, sizeof(uint32_t), cmp_u32);
}

/* Lloyd k-means (this project's definition; the reference calls `clump`):
 *   k_eff = min(k, n); centroids start at k_eff distinct seeded points;
 *   each iteration assigns every point (cosine: argmin 1 - dot; L2: argmin
 *   squared L2; lowest index wins ties), stops when no assignment changed,
 *   else replaces each non-empty centroid by the float64 mean of its members
 *   (members summed in index order), re-normalised for cosine
 *   (search.rs:55-62 rule); empty clusters keep their centroid.
 * Returns the number of centroid updates performed. */
long or_kmeans(const float *x, size_t n, size_t d, size_t k, int metric,
               uint64_t seed, size_t max_iter, float *centroids) {
    size_t ke = k < n ? k : n;
    if (ke == 0) return 0;
    uint32_t *init = (uint32_t *)malloc(ke * sizeof(uint32_t));
    draw_distinct(n, ke, seed, init);
    for (size_t c = 0; c < ke; c++) memcpy(centroids + c * d, x + (size_t)init[c] * d, d * sizeof(float));
    free(init);
    uint32_t *assign = (uint32_t *)malloc(n * sizeof(uint32_t));
    uint32_t *prev = (uint32_t *)malloc(n * sizeof(uint32_t));
    double *sums = (double *)malloc(ke * d * sizeof(double));
    uint64_t *counts = (uint64_t *)malloc(ke * sizeof(uint64_t));
    long updates = 0;
    for (size_t it = 0; it < max_iter; it++) {
        if (metric == 0) or_assign_cosine(x, n, centroids, ke, d, assign);
        else assign_l2(x, n, centroids, ke, d, assign);
        if (it > 0 && memcmp(assign, prev, n * sizeof(uint32_t)) == 0) break;
        memset(sums, 0, ke * d * sizeof(double));
        memset(counts, 0, ke * sizeof(uint64_t));
        for (size_t i = 0; i < n; i++) {
            double *s = sums + (size_t)assign[i] * d;
            const float *xi = x + i * d;
            for (size_t j = 0; j < d; j++) s[j] += (double)xi[j];
            counts[assign[i]]++;
        }
        for (size_t c = 0; c < ke; c++) {
            if (!counts[c]) continue;
            float *cc = centroids + c * d;
            for (size_t j = 0; j < d; j++) cc[j] = (float)(sums[c * d + j] / (double)counts[c]);
            if (metric == 0) or_normalize(cc, d, cc);
        }
        memcpy(prev, assign, n * sizeof(uint32_t));
        updates++;
    }
    free(assign);
    free(prev);
    free(sums);
    free(counts);
    return updates;
}

/* pq.rs:75-124 with this project's k-means: one squared-L2 k-means per
 * subspace of the rows x[n*d] (seed + m, max_iter).  Returns the codebook
 * size, min(K, n). */
static size_t pq_fit(const float *x, size_t n, size_t d, size_t M, size_t K,
                     uint64_t seed, size_t max_iter, float *codebooks) {
    size_t ds = d / M, Ke = K < n ? K : n;
    float *sub = (float *)malloc(n * ds * sizeof(float));
    for (size_t m = 0; m < M; m++) {
        for (size_t i = 0; i < n; i++) memcpy(sub + i * ds, x + i * d + m * ds, ds * sizeof(float));
        or_kmeans(sub, n, ds, Ke, 1, seed + m, max_iter, codebooks + m * Ke * ds);
    }
    free(sub);
    return Ke;
}

/* search.rs:546-787 with this project's k-means: training sample, cosine
 * coarse k-means (seed), list assignment of all vectors, residuals v - c,
 * one L2 k-means per subspace (seed + m, pq.rs:101-106) or, with use_opq,
 * OPQ training (opq.fit(training, count, 10), search.rs:732-749), then every
 * residual encoded (opq.quantize rotates it first, opq.rs:112-115).
 * `vectors` must already be normalised (add_slice rule).  Returns 0, or -1
 * on invalid shapes. */
int or_ivfpq_build(const float *vectors, size_t n, size_t d, size_t L,
                   size_t M, size_t K, uint64_t seed, size_t sample,
                   size_t max_iter, int use_opq, float *centroids,
                   float *codebooks, uint32_t *assign, uint8_t *codes,
                   float *rotation, size_t *K_actual) {
    if (n == 0 || M == 0 || d % M || K == 0 || K > 256 || n < K || max_iter == 0) return -1;
    size_t ds = d / M;
    size_t nt = (sample == 0 || sample >= n) ? n : sample;
    if (use_opq && nt < K) return -1;
    uint32_t *tidx = (uint32_t *)malloc(n * sizeof(uint32_t));
    or_sample_indices(n, sample, seed, tidx);
    float *train = (float *)malloc(nt * d * sizeof(float));
    for (size_t i = 0; i < nt; i++) memcpy(train + i * d, vectors + (size_t)tidx[i] * d, d * sizeof(float));
    size_t Le = L < nt ? L : nt;
    or_kmeans(train, nt, d, Le, 0, seed, max_iter, centroids);
    or_assign_cosine(vectors, n, centroids, Le, d, assign);
    float *res = (float *)malloc(n * d * sizeof(float));
    for (size_t i = 0; i < n; i++) {
        const float *c = centroids + (size_t)assign[i] * d;
        for (size_t j = 0; j < d; j++) res[i * d + j] = vectors[i * d + j] - c[j];
    }
    for (size_t i = 0; i < nt; i++) /* copy_rows_by_index, search.rs:737-745 */
        memcpy(train + i * d, res + (size_t)tidx[i] * d, d * sizeof(float));
    size_t Ke;
    if (use_opq) {
        or_opq_fit(train, nt, d, M, K, 10, seed, 100, rotation, codebooks, &Ke);
        float *rv = (float *)malloc(d * sizeof(float));
        for (size_t i = 0; i < n; i++) {
            or_matvec(rotation, res + i * d, d, rv);
            memcpy(res + i * d, rv, d * sizeof(float));
        }
        free(rv);
    } else {
        Ke = pq_fit(train, nt, d, M, K, seed, max_iter, codebooks);
    }
    or_pq_encode(codebooks, M, Ke, ds, res, n, codes);
    *K_actual = Ke;
    free(tidx);
    free(train);
    free(res);
    return 0;
}

/* ------------------------------------------------------------------------ */
/* OPQ (src/ivf_pq/opq.rs)                                                  */
/* ------------------------------------------------------------------------ */

/* matrix_vector_multiply, opq.rs:180-191: row i summed from 0.0 in order. */
void or_matvec(const float *R, const float *v, size_t d, float *out) {
    for (size_t i = 0; i < d; i++) {
        const float *row = R + i * d;
        float s = 0.0f;
        for (size_t j = 0; j < d; j++) s += row[j] * v[j];
        out[i] = s;
    }
}

/* transpose_matrix_vector_multiply, opq.rs:194-205. */
void or_matvec_t(const float *R, const float *v, size_t d, float *out) {
    for (size_t i = 0; i < d; i++) {
        float s = 0.0f;
        for (size_t j = 0; j < d; j++) s += R[j * d + i] * v[j];
        out[i] = s;
    }
}

/* The orthogonal polar factor of M (opq.rs:280-294 takes U V^T from an SVD).
 * One-sided Jacobi (Hestenes; Demmel & Veselic 1992) in float64: column pairs
 * of A = M are rotated until every pair is orthogonal to 1e-15, the rotations
 * accumulated in V, so A = U S.  Columns of norm <= 1e-12 of the largest
 * (M rank-deficient) are completed, in column order, by the unit vector with
 * the largest component outside the columns so far (Gram-Schmidt, two passes,
 * lowest index on ties).  R = U V^T rounded to float32. */
void or_polar(const float *Mf, size_t d, float *R) {
    /* A, V and U are stored transposed (column j is row j); every sum runs
     * over k in ascending order. */
    double *At = (double *)malloc(d * d * sizeof(double));
    double *Vt = (double *)calloc(d * d, sizeof(double));
    double *Ut = (double *)calloc(d * d, sizeof(double));
    double *S = (double *)calloc(d * d, sizeof(double));
    double *u = (double *)malloc(d * sizeof(double));
    double *best = (double *)malloc(d * sizeof(double));
    double *nrm = (double *)malloc(d * sizeof(double));
    char *ok = (char *)calloc(d, 1);
    for (size_t k = 0; k < d; k++)
        for (size_t j = 0; j < d; j++) At[j * d + k] = (double)Mf[k * d + j];
    for (size_t i = 0; i < d; i++) Vt[i * d + i] = 1.0;
    for (int sweep = 0; sweep < 64; sweep++) {
        int changed = 0;
        for (size_t p = 0; p + 1 < d; p++)
            for (size_t q = p + 1; q < d; q++) {
                double *ap = At + p * d, *aq = At + q * d;
                double a = 0.0, b = 0.0, g = 0.0;
                for (size_t k = 0; k < d; k++) {
                    double x = ap[k], y = aq[k];
                    a += x * x;
                    b += y * y;
                    g += x * y;
                }
                if (g == 0.0 || fabs(g) <= 1e-15 * sqrt(a * b)) continue;
                double z = (b - a) / (2.0 * g);
                double t = (z >= 0.0 ? 1.0 : -1.0) / (fabs(z) + sqrt(1.0 + z * z));
                double c = 1.0 / sqrt(1.0 + t * t), s = c * t;
                double *vp = Vt + p * d, *vq = Vt + q * d;
                for (size_t k = 0; k < d; k++) {
                    double x = ap[k], y = aq[k];
                    ap[k] = c * x - s * y;
                    aq[k] = s * x + c * y;
                }
                for (size_t k = 0; k < d; k++) {
                    double x = vp[k], y = vq[k];
                    vp[k] = c * x - s * y;
                    vq[k] = s * x + c * y;
                }
                changed = 1;
            }
        if (!changed) break;
    }
    double smax = 0.0;
    for (size_t j = 0; j < d; j++) {
        double s2 = 0.0;
        for (size_t k = 0; k < d; k++) s2 += At[j * d + k] * At[j * d + k];
        nrm[j] = sqrt(s2);
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
                    const double *uc = Ut + c * d;
                    double pr = 0.0;
                    for (size_t k = 0; k < d; k++) pr += uc[k] * u[k];
                    for (size_t k = 0; k < d; k++) u[k] -= pr * uc[k];
                }
            double s2 = 0.0;
            for (size_t k = 0; k < d; k++) s2 += u[k] * u[k];
            if (s2 > bn) {
                bn = s2;
                memcpy(best, u, d * sizeof(double));
            }
        }
        bn = sqrt(bn);
        for (size_t k = 0; k < d; k++) Ut[j * d + k] = best[k] / bn;
        ok[j] = 1;
    }
    /* R[i][j] = sum over k ascending of U[i][k] V[j][k] */
    for (size_t k = 0; k < d; k++)
        for (size_t i = 0; i < d; i++) {
            double ui = Ut[k * d + i];
            for (size_t j = 0; j < d; j++) S[i * d + j] += ui * Vt[k * d + j];
        }
    for (size_t i = 0; i < d * d; i++) R[i] = (float)S[i];
    free(At);
    free(Vt);
    free(Ut);
    free(S);
    free(u);
    free(best);
    free(nrm);
    free(ok);
}

/* OptimizedProductQuantizer::fit (opq.rs:65-109) with
 * compute_optimal_rotation (:232-295): R starts as the identity; each
 * iteration fits PQ on the rows rotated by R (the rows as given in the
 * first), then accumulates in float32, over the first min(n, 5000) rows in
 * order, M[i][j] += rec_i * x_j where rec = reconstruct(quantize(R x)), and
 * takes R = polar(M).  The codebooks are those of the last PQ fit, trained
 * under the rotation before the last update (as in the reference).  The
 * reference's PQ fits are unseeded (pq.rs:61-63); here each uses seed. */
int or_opq_fit(const float *data, size_t n, size_t d, size_t M, size_t K,
               size_t iterations, uint64_t seed, size_t max_iter,
               float *rotation, float *codebooks, size_t *K_actual) {
    if (n < K || M == 0 || d == 0 || d % M || iterations == 0) return -1;
    size_t ds = d / M, ns = n < 5000 ? n : 5000, Ke = 0;
    float *rot = (float *)malloc(n * d * sizeof(float));
    float *rv = (float *)malloc(d * sizeof(float));
    float *rec = (float *)malloc(d * sizeof(float));
    float *Mx = (float *)malloc(d * d * sizeof(float));
    uint8_t *code = (uint8_t *)malloc(M);
    memset(rotation, 0, d * d * sizeof(float));
    for (size_t i = 0; i < d; i++) rotation[i * d + i] = 1.0f;
    memcpy(rot, data, n * d * sizeof(float));
    for (size_t it = 0; it < iterations; it++) {
        if (it > 0)
            for (size_t i = 0; i < n; i++) or_matvec(rotation, data + i * d, d, rot + i * d);
        Ke = pq_fit(rot, n, d, M, K, seed, max_iter, codebooks);
        memset(Mx, 0, d * d * sizeof(float));
        for (size_t k = 0; k < ns; k++) {
            const float *x = data + k * d;
            or_matvec(rotation, x, d, rv);
            or_pq_encode(codebooks, M, Ke, ds, rv, 1, code);
            or_pq_reconstruct(codebooks, M, Ke, ds, code, rec);
            for (size_t i = 0; i < d; i++)
                for (size_t j = 0; j < d; j++) Mx[i * d + j] += rec[i] * x[j];
        }
        or_polar(Mx, d, rotation);
    }
    *K_actual = Ke;
    free(rot);
    free(rv);
    free(rec);
    free(Mx);
    free(code);
    return 0;
}

/* ------------------------------------------------------------------------ */
/* flat exact search                                                        */
/* ------------------------------------------------------------------------ */

typedef struct {
    const float *base, *queries;
    size_t n, d, nq, k;
    int metric;
    int64_t *out_ids;
    float *out_dists;
    size_t next;
} flat_job;

static void *flat_worker(void *arg) {
    flat_job *job = (flat_job *)arg;
    uint64_t *keys = (uint64_t *)malloc((job->n ? job->n : 1) * sizeof(uint64_t));
    for (;;) {
        size_t i = __atomic_fetch_add(&job->next, 1, __ATOMIC_RELAXED);
        if (i >= job->nq) break;
        const float *q = job->queries + i * job->d;
        for (size_t j = 0; j < job->n; j++) {
            const float *x = job->base + j * job->d;
            float dist = job->metric == 0 ? or_l2sq(q, x, job->d) : 1.0f - or_dot(q, x, job->d);
            keys[j] = cand_key(dist, (uint32_t)j);
        }
        size_t m = top_k_keys(keys, job->n, job->k);
        for (size_t j = 0; j < job->k; j++) {
            job->out_ids[i * job->k + j] = j < m ? (int64_t)(uint32_t)keys[j] : -1;
            job->out_dists[i * job->k + j] = j < m ? key_dist(keys[j]) : INFINITY;
        }
    }
    free(keys);
    return NULL;
}

/* Brute force top-k: metric 0 = squared L2 (distance.rs:78-83), metric 1 =
 * 1 - dot (distance.rs:104-109); ties by lower index. */
int or_flat_search(const float *base, size_t n, size_t d, const float *queries,
                   size_t nq, size_t k, int metric, int threads,
                   int64_t *out_ids, float *out_dists) {
    flat_job job = {base, queries, n, d, nq, k, metric, out_ids, out_dists, 0};
    int t = resolve_threads(threads);
    if ((size_t)t > nq) t = nq ? (int)nq : 1;
    pthread_t *tids = (pthread_t *)malloc((size_t)t * sizeof(pthread_t));
    for (int i = 0; i < t; i++) pthread_create(&tids[i], NULL, flat_worker, &job);
    for (int i = 0; i < t; i++) pthread_join(tids[i], NULL);
    free(tids);
    return 0;
}
