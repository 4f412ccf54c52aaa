/*
 * vicinity_gpu.h -- C ABI of the MI355X (gfx950) IVF-PQ search engine.
 *
 * This is the drop-in boundary for vicinity's IVF-PQ index
 * (src/ivf_pq/search.rs).  Every entry point names the reference interface it
 * replaces.  All arguments are plain pointers and sizes; host buffers are
 * owned by the caller and copied (inputs) or filled (outputs) before the call
 * returns.  No C++ exception crosses this boundary.
 *
 * Status codes map onto vicinity's RetrieveError (src/error.rs:17-80).  The
 * message of the last failure on the calling thread is vgpu_last_error().
 *
 * Threading: one handle may be searched from several threads at once, as the
 * reference's search(&self) may (src/ivf_pq/search.rs:1087): each call
 * borrows its own device workspace and, when it passes no stream, its own
 * stream.  add/build/load/setters wait for running searches and exclude new
 * ones, as the reference's &mut self methods do; free needs exclusive access.
 */
#ifndef VICINITY_GPU_H
#define VICINITY_GPU_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- status codes (src/error.rs:17-80) ----------------------------------- */
#define VGPU_OK 0
#define VGPU_ERR_EMPTY_INDEX 1        /* RetrieveError::EmptyIndex */
#define VGPU_ERR_INVALID_PARAMETER 2  /* RetrieveError::InvalidParameter */
#define VGPU_ERR_INVALID_CONFIG 3     /* RetrieveError::InvalidConfig */
#define VGPU_ERR_NOT_BUILT 4          /* RetrieveError::NotBuilt */
#define VGPU_ERR_ALREADY_BUILT 5      /* RetrieveError::AlreadyBuilt */
#define VGPU_ERR_UNSUPPORTED 6        /* RetrieveError::Unsupported */
#define VGPU_ERR_DIMENSION_MISMATCH 7 /* RetrieveError::DimensionMismatch */
#define VGPU_ERR_DEVICE 8             /* HIP runtime failure (RetrieveError::Other) */
#define VGPU_ERR_OUT_OF_MEMORY 9      /* device allocation failed (RetrieveError::Other) */

/* Scan arithmetic.  Both modes return the oracle's bit-exact distances:
 *   FAST  ranks candidates with a per-query decomposed table
 *         (||q-c||^2 + b(x) - 2 q.cw), then rescores the survivors with the
 *         reference's residual-table arithmetic (pq.rs:232-251) and falls
 *         back to EXACT for a query whose margin check fails;
 *   EXACT builds the reference's per-(query, list) residual table. */
#define VGPU_MODE_FAST 0
#define VGPU_MODE_EXACT 1

/* IVFPQParams (src/ivf_pq/search.rs:284-312).  use_opq != 0 trains OPQ at
 * build (opq.rs:65-109) for dimension <= 2048; searches then scan in EXACT
 * mode on rotated residual tables. */
typedef struct vgpu_ivfpq_params {
    size_t num_clusters;  /* nlist */
    size_t nprobe;        /* default probes per query */
    size_t num_codebooks; /* M, must divide the dimension */
    size_t codebook_size; /* ksub, 1..=256; 16 selects 4-bit FastScan */
    uint64_t seed;        /* k-means seed */
    int use_opq;
} vgpu_ivfpq_params;

typedef struct vgpu_ivfpq_info {
    size_t dimension, num_vectors, num_clusters, nprobe, num_codebooks, codebook_size;
    size_t subvector_dim;
    int built, has_vectors, mode;
} vgpu_ivfpq_info;

/* Per-call device timings (ms, hipEvents on the call's stream) and
 * counters of the search that finished last on a handle. */
typedef struct vgpu_search_stats {
    float ms_normalize, ms_coarse, ms_select, ms_scan, ms_fallback, ms_rerank, ms_total;
    uint64_t candidates;     /* sum over queries of scanned list entries */
    uint64_t scan_bytes;     /* algorithmic bytes of the scan: candidates * (code bytes + 4) */
    uint32_t fallback_queries; /* FAST queries recomputed in EXACT mode */
    uint32_t coarse_overflow;  /* queries whose probe selection took the exact fallback */
    uint32_t nq;
    uint64_t fast_flushes;     /* FAST: buffer flushes summed over queries */
    uint64_t fast_appends;     /* FAST: entries that passed the running threshold */
    uint32_t fallback_ties;    /* FAST fallbacks caused by more equal distances than the buffer holds */
    uint32_t fast_retries;     /* FAST queries that needed a second pass over their lists */
    float ms_table;            /* FAST: the per-query table pre-pass (not part of ms_scan) */
} vgpu_search_stats;

typedef struct vgpu_ivfpq vgpu_ivfpq;

const char *vgpu_last_error(void);
/* 1 when a gfx950 device is visible, 0 otherwise (never initialises work). */
int vgpu_device_available(void);

/* IVFPQIndex::new (search.rs:382-405).  Uses the current HIP device. */
int vgpu_ivfpq_new(size_t dimension, const vgpu_ivfpq_params *params, vgpu_ivfpq **out);
void vgpu_ivfpq_free(vgpu_ivfpq *h);

/* IVFPQIndex::add_slice (search.rs:488-512) for n rows: each row is
 * L2-normalised on insert; doc_ids[i] is returned by search. */
int vgpu_ivfpq_add(vgpu_ivfpq *h, const uint32_t *doc_ids, const float *vectors, size_t n);

/* IVFPQIndex::build_with_training_options (search.rs:534-544):
 * training_sample_size 0 = train on every vector.  k-means runs its
 * assignment steps on the GPU. */
int vgpu_ivfpq_build(vgpu_ivfpq *h, size_t training_sample_size, size_t kmeans_max_iter);

/* Upload an index built elsewhere (the reference's build() or
 * load_from_dir(), search.rs:1034-1084): centroids f32[L*d], codebooks
 * f32[M*K*ds], list_offsets u64[L+1], list_ids u32[n] (insertion indices,
 * ascending inside a list), codes u8[n*M] in insertion order
 * (quantized_codes), doc_ids u32[n] or NULL (identity), vectors f32[n*d]
 * normalised or NULL (no rerank).  Marks the index built. */
int vgpu_ivfpq_load(vgpu_ivfpq *h, const float *centroids, size_t num_centroids,
                    const float *codebooks, size_t codebook_size,
                    const uint64_t *list_offsets, const uint32_t *list_ids,
                    const uint8_t *codes, const uint32_t *doc_ids, const float *vectors,
                    size_t num_vectors);

int vgpu_ivfpq_set_nprobe(vgpu_ivfpq *h, size_t nprobe); /* search.rs:342-348 */
int vgpu_ivfpq_set_mode(vgpu_ivfpq *h, int mode);
int vgpu_ivfpq_compact(vgpu_ivfpq *h);                  /* search.rs compact() */
int vgpu_ivfpq_get_info(const vgpu_ivfpq *h, vgpu_ivfpq_info *out);

/* IVFPQIndex::search (search.rs:1087-1093): up to k (doc_id, distance)
 * pairs, ascending; *out_len receives the count. */
int vgpu_ivfpq_search(vgpu_ivfpq *h, const float *query, size_t dim, size_t k,
                      uint32_t *out_ids, float *out_dists, size_t *out_len);
/* IVFPQIndex::search_reranked (search.rs:1117-1158): distances are exact
 * cosine distances 1 - q.v. */
int vgpu_ivfpq_search_reranked(vgpu_ivfpq *h, const float *query, size_t dim, size_t k,
                               size_t pool, uint32_t *out_ids, float *out_dists, size_t *out_len);

/* Batch search, the shape of PyIVFPQIndex.batch_search (python.rs:744-793)
 * and HNSW's search_batch (src/hnsw/graph.rs:2716-2768): queries f32[nq*dim]
 * row-major (dim != the index dimension -> DimensionMismatch, search.rs:1188-1193);
 * nprobe 0 = the index default; rerank_pool 0 = no rerank.
 * Output rows (nq, k), padded with (-1, +inf) (python.rs:778-785). */
int vgpu_ivfpq_search_batch(vgpu_ivfpq *h, const float *queries, size_t nq, size_t dim, size_t k,
                            size_t nprobe, size_t rerank_pool, int64_t *out_ids,
                            float *out_dists);
/* Same with device pointers on `stream` (a hipStream_t; NULL = the stream
 * of the call's borrowed workspace); returns after the search completes.
 * A query holding a NaN or an infinity is VGPU_ERR_INVALID_PARAMETER, as in
 * vgpu_ivfpq_search_batch; the other rows of the batch are still written, and
 * the offending rows are padding (-1, +inf). */
int vgpu_ivfpq_search_batch_device(vgpu_ivfpq *h, const float *d_queries, size_t nq,
                                   size_t dim, size_t k, size_t nprobe, size_t rerank_pool,
                                   int64_t *d_out_ids, float *d_out_dists, void *stream);
/* No counterpart in the reference: for callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc).  vgpu_ivfpq_search_batch_device without any device or
 * pinned-host allocation: the workspace is a 64 MiB device array inside the library (one
 * per GPU, held until the process ends), and a batch goes in query chunks
 * that fit it; a shape whose single query does not fit (about 2.5 KB per
 * query at d 128, nprobe 32, k 100) is VGPU_ERR_INVALID_PARAMETER.  Every
 * call on one GPU shares that array, whatever the handle: the library holds a
 * per-GPU lock across each call, so synchronous calls from several threads
 * take turns.  The index's device must be current.  stream NULL = the
 * handle's own stream; returns after the search completes; does not update
 * vgpu_ivfpq_last_stats or the profiling timers.  Non-finite queries as for
 * vgpu_ivfpq_search_batch_device.
 * Under stream capture (hipStreamIsCapturing) the call records its kernels
 * and returns without waiting: completion is the caller's, a non-finite query
 * shows only as a padding row, and replays of captured graphs that overlap
 * each other or another call on the same GPU race (the lock covers recording,
 * not replay).  The first call on a GPU (which looks up the array's address)
 * must not be under capture. */
int vgpu_ivfpq_search_batch_device_noalloc(vgpu_ivfpq *h, const float *d_queries, size_t nq,
                                           size_t dim, size_t k, size_t nprobe,
                                           size_t rerank_pool, int64_t *d_out_ids,
                                           float *d_out_dists, void *stream);
int vgpu_ivfpq_last_stats(const vgpu_ivfpq *h, vgpu_search_stats *out);
/* hipEvent timing of later search calls, read back by vgpu_ivfpq_last_stats:
 * 0 off (default); 1 every phase (events around each stage, one host wait per
 * query chunk); 2 the scan kernels only (two events per chunk, read after the
 * call's final wait; the other phase times read 0). */
int vgpu_ivfpq_set_profiling(vgpu_ivfpq *h, int enabled);

/* Filtered search.  IVFPQIndex::with_filtering (search.rs:413-435): switch
 * per-document categories on, before build (VGPU_ERR_ALREADY_BUILT after). */
int vgpu_ivfpq_enable_filtering(vgpu_ivfpq *h);
/* IVFPQIndex::add_metadata (search.rs:439-475), the filter field only: the
 * document's category 0..63, or -1 when its metadata lacks the field (it then
 * never matches).  Outside -1..63: VGPU_ERR_INVALID_PARAMETER; filtering off:
 * VGPU_ERR_UNSUPPORTED.  Lists keep the categories their members had at build
 * time in their bitmasks (search.rs:626-648); matching reads the current ones. */
int vgpu_ivfpq_set_category(vgpu_ivfpq *h, uint32_t doc_id, int64_t category);
/* IVFPQIndex::search_with_filter (search.rs:1407-1549) with
 * MetadataFilter::Equals(filter field, Int(category)): up to k (doc_id,
 * distance) pairs of documents carrying the category, ascending; the probe
 * widens to every list when the probed ones hold fewer than k matches.
 * Distances use the reference's table arithmetic for every ksub. */
int vgpu_ivfpq_search_filtered(vgpu_ivfpq *h, const float *query, size_t dim, size_t k,
                               int64_t category, uint32_t *out_ids, float *out_dists,
                               size_t *out_len);

/* search_with_filter for a batch: query i restricted to categories[i]
 * (0..63), rows (nq, k) padded with (-1, +inf) like search_batch
 * (python.rs:778-785).  The reference has the one-query form only
 * (search.rs:1407-1549); each row equals that query's
 * vgpu_ivfpq_search_filtered result. */
int vgpu_ivfpq_search_filtered_batch(vgpu_ivfpq *h, const float *queries, size_t nq, size_t dim,
                                     size_t k, const int64_t *categories, int64_t *out_ids,
                                     float *out_dists);

/* The lists' category bitmasks, masks u64[L] (L = the built index's list
 * count).  No counterpart in the reference's API: they carry
 * Cluster::filter_bitmask (src/ivf_pq/cluster.rs:24-27) through the snapshot
 * files, which persist it in clusters.bin (persistence.rs:51-68, :195-248);
 * set replaces the bitmasks taken at build or load time. */
int vgpu_ivfpq_get_list_masks(const vgpu_ivfpq *h, uint64_t *masks, size_t L);
int vgpu_ivfpq_set_list_masks(vgpu_ivfpq *h, const uint64_t *masks, size_t L);

/* OPQ rotation R, f32[d*d] row-major (OptimizedProductQuantizer::rotation,
 * src/ivf_pq/opq.rs:37-38; read by rotation_matrix :151-153).  get writes it
 * and sets *present = 1, or sets *present = 0 for an index without one
 * (Quantizer::Product, or OPQ never trained).  set gives an index made with
 * use_opq the rotation of an index built elsewhere, before vgpu_ivfpq_load
 * (the Quantizer::Optimized of a snapshot, search.rs:1034-1084); R = NULL
 * clears it.  Searches then table R (q - c) (opq.rs:120-123). */
int vgpu_ivfpq_get_rotation(const vgpu_ivfpq *h, float *R, size_t len, int *present);
int vgpu_ivfpq_set_rotation(vgpu_ivfpq *h, const float *R, size_t len);

/* The probed lists of each query in probe order (search.rs:1602-1617),
 * lists u32[nq*nprobe]; returns the probe count per query in *out_p. */
int vgpu_ivfpq_probe_batch(vgpu_ivfpq *h, const float *queries, size_t nq, size_t dim,
                           size_t nprobe, uint32_t *lists, size_t *out_p);

/* Copy the built artifacts back (any pointer may be NULL): same layouts as
 * vgpu_ivfpq_load; codes in insertion order. */
int vgpu_ivfpq_export(const vgpu_ivfpq *h, float *centroids, float *codebooks,
                      uint64_t *list_offsets, uint32_t *list_ids, uint8_t *codes,
                      uint32_t *doc_ids, float *vectors);

/* IVFPQIndex::reconstruct (search.rs:857-884): the vector the codes of
 * insertion index idx approximate, out f32[d]: the decoded residual
 * (pq.rs:284-290; OPQ: R^T of it, opq.rs:134-139) plus the centroid of the
 * list holding idx.  Works after compact().  VGPU_ERR_INVALID_PARAMETER when
 * not built or idx >= num_vectors. */
int vgpu_ivfpq_reconstruct(const vgpu_ivfpq *h, size_t idx, float *out, size_t len);

/* IVFPQIndex::memory_usage (search.rs:1552-1577, MemoryReport in
 * src/memory.rs): host bytes by the reference's categories (raw vectors;
 * graph, always 0; codes and quantizer; doc ids, centroids and lists), plus
 * the HBM the index and its search workspaces hold. */
typedef struct {
    size_t vectors_bytes, graph_bytes, quantized_bytes, metadata_bytes;
    size_t device_bytes;
} vgpu_memory_report;
int vgpu_ivfpq_memory_usage(const vgpu_ivfpq *h, vgpu_memory_report *out);

/* ---- file-backed search: IVFPQFileSearcher (src/ivf_pq/search.rs:247-282,
 * :1620-2041) --------------------------------------------------------------
 * The routing metadata in memory (what load_from_parts, search.rs:1679-1762,
 * parses from the snapshot: centroids, codebooks, the clusters as
 * list_offsets/list_ids, doc ids, the OPQ rotation or NULL); the PQ codes
 * (list_codes.bin + list_offsets.bin, else codes.bin) and raw_vectors.bin
 * stay in the snapshot directory `dir` and are read per search call.  A
 * call probes with the full index's centroids, reads the codes of the union
 * of the probed lists into HBM and scans them there; a reranked call reads
 * the raw vectors of the approximate candidates only.  Results equal the
 * in-memory index's on the same snapshot.  One call at a time per handle. */
typedef struct vgpu_ivfpq_file vgpu_ivfpq_file;
/* IVFPQFileSearchDiagnostics (search.rs:263-282), per query. */
typedef struct vgpu_file_diagnostics {
    uint64_t probed_lists, scanned_vectors, code_reads, code_bytes, retained_candidates,
        raw_vector_reads, raw_vector_bytes, reranked_candidates;
} vgpu_file_diagnostics;
int vgpu_ivfpq_file_open(size_t dimension, const vgpu_ivfpq_params *params, const float *centroids,
                         size_t num_centroids, const float *codebooks, size_t codebook_size,
                         const uint64_t *list_offsets, const uint32_t *list_ids,
                         const uint32_t *doc_ids, size_t num_vectors, const float *rotation,
                         const char *dir, int raw_vectors_present, vgpu_ivfpq_file **out);
void vgpu_ivfpq_file_free(vgpu_ivfpq_file *h);
int vgpu_ivfpq_file_set_nprobe(vgpu_ivfpq_file *h, size_t nprobe); /* search.rs:1765-1768 */
/* search / search_reranked / batch of them (search.rs:1800-1891): nprobe 0 =
 * the searcher's, rerank_pool 0 = no rerank; rows padded with (-1, +inf);
 * diag (NULL allowed) receives nq rows. */
int vgpu_ivfpq_file_search_batch(vgpu_ivfpq_file *h, const float *queries, size_t nq, size_t dim,
                                 size_t k, size_t nprobe, size_t rerank_pool, int64_t *out_ids,
                                 float *out_dists, vgpu_file_diagnostics *diag);
/* File reads of the last search call (positional reads and bytes). */
int vgpu_ivfpq_file_last_io(const vgpu_ivfpq_file *h, uint64_t *reads, uint64_t *bytes);

/* ---- flat exact search (src/distance.rs:78-109) ---------------------------
 * metric 0: squared L2 ||q||^2 - 2 q.x + ||x||^2 ranking, distances rescored
 * with l2_distance_squared; metric 1: 1 - q.x (cosine_distance_normalized). */
typedef struct vgpu_flat vgpu_flat;
int vgpu_flat_new(size_t dimension, int metric, vgpu_flat **out);
void vgpu_flat_free(vgpu_flat *h);
int vgpu_flat_add(vgpu_flat *h, const float *vectors, size_t n);
int vgpu_flat_search_batch(vgpu_flat *h, const float *queries, size_t nq, size_t dim, size_t k,
                           int64_t *out_ids, float *out_dists);
int vgpu_flat_search_batch_device(vgpu_flat *h, const float *d_queries, size_t nq, size_t dim,
                                  size_t k, int64_t *d_out_ids, float *d_out_dists, void *stream);
/* Device time of the last search: ms_gemm the ranking kernel (bf16x3 MFMA
 * for d <= 128 and k <= 32, fp32 MFMA otherwise), ms_total ranking through
 * merge, exact rescoring, fallback and output. */
int vgpu_flat_last_ms(const vgpu_flat *h, float *ms_gemm, float *ms_total);
/* Queries of the last flat search whose kept candidates could not be proved
 * to hold the exact top-k; the database slices that could hide a result were
 * then scanned exhaustively with the exact arithmetic (their results are
 * exact either way). */
int vgpu_flat_last_fallbacks(const vgpu_flat *h, uint32_t *queries);

/* ---- per-kernel test entry points (host buffers) -------------------------- */
/* Host steps of the build, no device needed.  Inverted lists from list
 * labels (search.rs:624-657): offsets u64[L+1], list_ids u32[n]; a label >= L
 * (what a faulty device would return) is VGPU_ERR_DEVICE. */
int vgpu_test_host_lists(const uint32_t *assign, size_t n, size_t L, uint64_t *offsets,
                         uint32_t *list_ids);
/* The host cosine k-means update of centroids f32[k*d] in place (float64
 * member means in row order, re-normalised; empty keys keep their row); a
 * label >= k is VGPU_ERR_DEVICE. */
int vgpu_test_host_centroid_update(const float *x, size_t n, size_t d, const uint32_t *assign,
                                   size_t k, float *centroids);
/* The OPQ polar factor U V^T of M f32[d*d] (compute_optimal_rotation,
 * opq.rs:280-294) into R f32[d*d]. */
int vgpu_test_polar_factor(const float *m, size_t d, float *r);
/* The error bounds behind the exactness proofs, evaluated on the host by
 * the same code the kernels run (test hooks with no reference counterpart;
 * no device call): FAST ranking value against the ADC distance
 * (search.rs:1318-1354), bf16x3 and fp32 coarse scores against the
 * sequential dot (search.rs:1602-1617), flat bf16x3 key against
 * l2_distance_squared / 1 - dot (distance.rs:78-109). */
int vgpu_test_bound_fast_tau(size_t d, size_t M, size_t ds, float qn, float cmax, float rmax,
                             float t0max, float *out);
int vgpu_test_bound_coarse(size_t d, float qn, float cmax, float *out_bf16x3, float *out_fp32);
int vgpu_test_bound_flat(size_t d, int metric, float qn, float xn, int ib, float *out);
/* Device-allocation failure injection (a test hook with no reference
 * counterpart): after `after` more device allocations by the library succeed,
 * the next `count` fail with VGPU_ERR_OUT_OF_MEMORY, as hipMalloc's
 * out-of-memory would (the reference's allocation failure is a process
 * abort).  count 0 disarms.  Process-wide. */
int vgpu_test_fail_device_allocations(size_t after, size_t count);
/* Bound on the rotated residuals (floats) one pass of a filtered search
 * under OPQ holds; queries beyond it go in further passes (default 2^28). */
int vgpu_test_set_rres_limit(vgpu_ivfpq *h, size_t floats);
/* compute_adc_table_into (pq.rs:196-266) for nr residuals: tables f32[nr*M*K]. */
int vgpu_test_adc_tables(const float *codebooks, size_t M, size_t K, size_t ds,
                         const float *residuals, size_t nr, float *tables);
/* quantize (pq.rs:136-161) of n vectors: codes u8[n*M]. */
int vgpu_test_pq_encode(const float *codebooks, size_t M, size_t K, size_t ds,
                        const float *x, size_t n, uint8_t *codes);
/* normalize (search.rs:55-62) of n rows. */
int vgpu_test_normalize(const float *x, size_t n, size_t d, float *out);
/* quantize_lut_flat + fastscan_batch_flat (pq_simd.rs:576-769) of one
 * packed list (pq_simd.rs:426-486 layout): out f32[n]. */
int vgpu_test_fastscan(const uint8_t *packed, size_t n, size_t M, const float *lut, float *out);
/* Coarse dot products Q.C^T with the MFMA kernel: out f32[nq*L]. */
int vgpu_test_coarse_dots(const float *q, size_t nq, const float *c, size_t L, size_t d,
                          float *out);
/* The same products with the search path's split-bfloat16 (bf16x3) MFMA
 * kernel, d <= 128: out f32[nq*L]. */
int vgpu_test_coarse_dots_bf16x3(const float *q, size_t nq, const float *c, size_t L, size_t d,
                                 float *out);

#ifdef __cplusplus
}
#endif
#endif
