// Host-side launchers of the gfx950 kernels (one .hip file per kernel family).
// Shapes are validated by the callers in vgpu_index.cpp before any launch.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "vgpu_device.h"

namespace vgpu {

// Raise a kernel's dynamic-LDS limit to at least `bytes`; the attribute is set
// once per kernel and size increase, not on every launch.
void ensure_dyn_lds(const void* kernel, size_t bytes);

// HBM-resident IVF-PQ index (all pointers are device memory).
struct DevIndex {
    int d = 0, L = 0, M = 0, K = 0, ds = 0;
    uint32_t n = 0;
    const float* centroids = nullptr;  // [L*d] row-major
    const uint4* cb16 = nullptr;       // bf16 hi/lo centroid chunks (launch_coarse_bf16_pack)
    const float* codebooks = nullptr;  // [M*K*ds] codebook, codeword, dim
    const uint32_t* offsets = nullptr; // [L+1] list l = positions [off[l], off[l+1])
    const uint32_t* list_ids = nullptr;// [n] insertion index at each position
    const uint8_t* codes = nullptr;    // [n*M] codes at each position (list-major rows)
    const float* bias = nullptr;       // [n] ||x_r||^2 + 2 c.x_r at each position (K != 16)
    const uint32_t* doc_ids = nullptr; // [n] by insertion index
    const float* vectors = nullptr;    // [n*d] by insertion index, normalised (may be null)
    const uint8_t* packed = nullptr;   // FastScan blocks of every list (K == 16)
    const uint32_t* pack_off = nullptr;// [L+1] block offset of each list (K == 16)
    // Transposed 16-entry blocks of every list for the FAST scan (K == 256,
    // M a multiple of 16; null otherwise).  Block b of list l is block
    // tblk_off[l] + b; lane record m of block B (index 16 B + m) is M bytes of
    // tcodes, the 16 codes of codebooks m, m + 16, ... (byte j the code of
    // entry j ^ m), and one float of tbias, b(x) of entry m.  Entries past
    // the end of the list have code 0 and b(x) NaN.
    const uint8_t* tcodes = nullptr;
    const float* tbias = nullptr;
    const uint32_t* tblk_off = nullptr;// [L+1]
    uint32_t tblk_count = 0;           // blocks (one of slack past the last list's)
    float cmax = 0.f;                  // max ||c||
    float rmax = 0.f;                  // max ||decoded residual||
};

struct ScanArgs {
    const float* qn = nullptr;      // [nq*d] normalised queries
    const float* qnorm = nullptr;   // [nq] ||q_n||
    const uint32_t* probe = nullptr;// [nq*P] probed lists, probe order
    int nq = 0, P = 0;
    int kout = 0;                   // results kept per query (k, or the rerank pool)
    int kk = 0;                     // FAST: entries a flush keeps (> kout); EXACT: kout
    int exact = 0;                  // 1 = EXACT mode
    int only_flagged = 0;           // EXACT: run the queries of flag_list only
    uint32_t* flag_list = nullptr;  // [nq] queries FAST could not prove (appended by FAST)
    uint32_t* flag_count = nullptr; // entries of flag_list (zeroed by launch_finish)
    uint32_t* out_vidx = nullptr;   // [nq*kout] insertion indices, 0xffffffff padding
    float* out_dist = nullptr;      // [nq*kout]
    // Final rows instead (no rerank, kout = k): doc ids (insertion indices
    // when doc_ids is null) with (-1, +inf) padding, python.rs:778-785.
    int64_t* out_ids = nullptr;     // [nq*kout]
    float* out_dists = nullptr;     // [nq*kout]
    const uint32_t* doc_ids = nullptr;
    // Per-query statistics, one row of QSTAT_WORDS per query, written with plain
    // stores (no global atomics): [0] list entries scanned, [1] FAST flushes,
    // [2] FAST appends, [3] bit 0: FAST could not prove the query (rerun by the
    // EXACT kernel), bit 1: because of more equal distances than its buffer holds,
    // bit 2: FAST needed its second pass.
    uint32_t* qstat = nullptr;
    // OPQ: the rotated residual R (q - c) of every (query, slot), [nq*P*d];
    // null: the residual q - c (Quantizer::Product).  EXACT, filtered and
    // FastScan kernels only.
    const float* rres = nullptr;
    // FAST scan with 16 codebooks on transposed blocks: the per-query tables
    // written by launch_t2_tables ([nq][M * 256], the scan's LDS layout);
    // null: the scan builds each query's table itself.
    const float* t2 = nullptr;
};

// Writes result j of query q from a (distance, insertion index) key, or
// padding when !valid: the final (doc id, distance) row when a.out_ids is set,
// else the (insertion index, distance) row for a later rerank.
__device__ __forceinline__ void scan_emit(const ScanArgs& a, int q, int j, uint64_t key, bool valid) {
    const size_t o = (size_t)q * a.kout + j;
    const uint32_t v = (uint32_t)key;
    const float dist = valid ? key_dist(key) : __int_as_float(0x7f800000);
    if (a.out_ids) {
        a.out_ids[o] = valid ? (int64_t)(a.doc_ids ? a.doc_ids[v] : v) : (int64_t)-1;
        a.out_dists[o] = dist;
    } else {
        a.out_vidx[o] = valid ? v : 0xffffffffu;
        a.out_dist[o] = dist;
    }
}

// qbad / nbad (optional): per-row non-finite marks and their count; such a
// row is normalised as the zero vector.
void launch_normalize(const float* x, float* out, float* norms, int n, int d, hipStream_t s,
                      uint32_t* qbad = nullptr, unsigned int* nbad = nullptr);
void launch_coarse_dots(const float* Q, const float* C, float* D, int nq, int L, int d,
                        hipStream_t s);
// Probe selection with exact rescoring: probe[q*P..] = the P lists of smallest
// 1 - dot (ties: lower list index), ascending.  D may be overwritten for
// degenerate rows.  flag_list [nq] / flag_count [1]: device scratch; *flag_count
// must be 0 on entry and is left holding the number of degenerate rows.
// Probe selection of more than 1024 lists (up to SEL_WIDE_MAX): exact scores of
// every list into D (nq x L), then the P smallest (score, list) in order.
#define SEL_WIDE_MAX 16384
void launch_coarse_select_wide(float* D, const float* qn, const float* C, int nq, int L, int d, int P,
                               uint32_t* probe, hipStream_t s);
void launch_coarse_select(float* D, const float* qn, const float* qnorm, const float* C,
                          int nq, int L, int d, int P, float cmax, uint32_t* probe,
                          unsigned int* overflow, uint32_t* flag_list, uint32_t* flag_count,
                          hipStream_t s);

// ---- fused coarse quantiser (k_coarse_fused.hip): d <= 128, 1 <= P <= 64.
bool coarse_fused_supported(int d, int P);
// bf16 hi/lo copy of the centroids: L * ceil(d/32) * 8 uint4.
// uint4 chunks of the packed centroids (L padded to whole pipeline stages).
size_t coarse_bf16_pack_chunks(int L, int d);
void launch_coarse_bf16_pack(const float* C, int L, int d, uint4* Cb, hipStream_t s);
// Normalise the raw queries Q (or use them as given, normalize = 0) into qn /
// qnorm (either may be null), take each query's candidate lists by bf16x3
// MFMA scores and write probe[q][0..P) from them by exact score (C: the
// float32 centroids): the P lists of smallest reference score, in ascending
// order when `ordered`, else in no set order (what a scan needs); a query
// whose candidates may be incomplete is appended to flag_list (*flag_count
// must be 0 on entry) for launch_coarse_exact_flagged.  qbad / nbad as for
// launch_normalize.
void launch_coarse_fused(const float* Q, int nq, int d, const uint4* Cb, int L, float cmax, int P,
                         int normalize, int ordered, float* qn, float* qnorm, const float* C, uint32_t* probe,
                         uint32_t* flag_list, uint32_t* flag_count, hipStream_t s, uint32_t* qbad = nullptr,
                         unsigned int* nbad = nullptr);
// Exact probe selection for the flagged queries (dot products in LDS).
// fdots (COARSE_FLAG_PAR rows of L floats) and fdone (COARSE_FLAG_PAR zeroed
// counters) spread the first flagged queries' dot products over the grid;
// null: one workgroup per flagged query.
#define COARSE_FLAG_PAR 64
void launch_coarse_exact_flagged(const float* qn, const float* qnorm, const float* C, int nq, int L,
                                 int d, int P, float cmax, uint32_t* probe, unsigned int* overflow,
                                 const uint32_t* flag_list, const uint32_t* flag_count, hipStream_t s,
                                 float* fdots = nullptr, uint32_t* fdone = nullptr);
// Test entry: D[q][c] = Q[q] . C[c] with the fused kernel's bf16x3 MFMA.
void launch_coarse_bf16x3_dots(const float* Q, int nq, int d, const uint4* Cb, int L, float* D,
                               hipStream_t s);

size_t scan8_lds_bytes(const DevIndex& ix, const ScanArgs& a);
void launch_scan8_exact(const DevIndex& ix, const ScanArgs& a, hipStream_t s);
// search_with_filter: a.probe holds a.P list slots per query (slots >= L are
// padding), ecat[n] the category byte of each list-major entry (0xff: none),
// want[nq] each query's category; writes a.out_vidx / a.out_dist like EXACT
// mode (a.kk == a.kout), no statistics rows.
void launch_scan8_filtered(const DevIndex& ix, const ScanArgs& a, const uint8_t* ecat,
                           const uint8_t* want, hipStream_t s);
// FAST mode: per-query decomposed table, threshold buffer, exact rescoring of
// the provable candidate set; an unprovable query sets bit 0 of its qstat
// fallback word.
size_t scan8_fast_lds_bytes(const DevIndex& ix, const ScanArgs& a);
// t0 / t1 (optional): events the kernel's own dispatch records at its start
// and end (hipExtLaunchKernelGGL), so timing adds no marker packets.
void launch_scan8_fast(const DevIndex& ix, const ScanArgs& a, hipStream_t s, hipEvent_t t0 = nullptr,
                       hipEvent_t t1 = nullptr);

#define QSTAT_WORDS 4
// Search statistics: entries scanned, fallbacks, flushes, appends, fallbacks
// from ties, second passes; counter i lives at counters[i * COUNTER_STRIDE]
// (separate cache lines for the per-workgroup atomics); the counter after them
// (index NUM_SCAN_COUNTERS) counts queries sent to the exact coarse fallback.
#define NUM_SCAN_COUNTERS 6
#define COUNTER_STRIDE 8
// Chunk epilogue: doc-id mapping and padding of (vidx, dist)[nq][kin] into
// (out_ids, out_dists)[nq][k]; counters += the qstat rows (qstat may be null);
// *flag_count = *cflag_count = 0 (either may be null).  Rows q with
// qbad[q] != 0 (a non-finite query; qbad may be null) become padding.
void launch_finish(const uint32_t* vidx, const float* dist, const uint32_t* doc_ids, int nq, int kin,
                   int k, int64_t* out_ids, float* out_dists, const uint32_t* qstat,
                   unsigned long long* counters, uint32_t* flag_count, uint32_t* cflag_count,
                   hipStream_t s, const uint32_t* qbad = nullptr);
size_t fastscan_lds_bytes(const DevIndex& ix, const ScanArgs& a);
void launch_fastscan(const DevIndex& ix, const ScanArgs& a, hipStream_t s);

// Exact rerank of the scan's pool: 1 - q.v over stored vectors
// (search.rs:1148-1156), top-k by (distance, insertion index).
// Largest rerank pool (the pool's keys sit in LDS).
#define RERANK_MAX 8192
void launch_rerank(const DevIndex& ix, const float* qn, int nq, const uint32_t* pool_vidx,
                   int pool, int k, uint32_t* out_vidx, float* out_dist, hipStream_t s);
// The same over rows of a given vector array (pool_rows index it; ties go to
// the lower row): the file-backed searcher's candidate vectors.
void launch_rerank_vectors(const float* vectors, int d, const float* qn, int nq, const uint32_t* pool_rows,
                           int pool, int k, uint32_t* out_rows, float* out_dist, hipStream_t s);
// Zero n 64-bit words on stream s (a kernel, graph-capture safe).
void launch_zero_words(unsigned long long* p, size_t n, hipStream_t s);
// Map insertion indices to doc ids and pad with (-1, +inf) (python.rs:778-785).
void launch_finalize(const uint32_t* vidx, const float* dist, const uint32_t* doc_ids, int nq,
                     int kin, int k, int64_t* out_ids, float* out_dists, hipStream_t s);

// Build side.
// codes[i*M + m] = argmin_k ||x_i,m - c_{assign_i},m - cw_mk||^2 (pq.rs:136-161);
// centroids/assign may be null (x is then the residual itself).
// ---- OPQ (k_opq.hip) ----
// out[r] = R x_r (row-major R, d x d), x_r = X[r / xdiv] - C[lists[r]] when C is
// given (zero for lists[r] >= L), else X[r]; n rows.
void launch_rotate_rows(const float* R, const float* X, int xdiv, const float* C,
                        const uint32_t* lists, int L, size_t n, int d, float* out, hipStream_t s);
size_t rotate_rows_lds_bytes(int d);
// Mx[d*d] = sum over the first ns rows of reconstruct(codes[k])^T X[k] (float32, in order).
void launch_procrustes(const uint8_t* codes, const float* cb, int M, int K, int ds, const float* X,
                       int ns, int d, float* Mx, hipStream_t s);

// k-means update of every key (M subspaces x K, or M = 1): float64 member sums in
// row order, mean cast to float, optionally normalised; empty keys keep their
// row; subspaces with active[m] == 0 are skipped (active may be null).  u8:
// labels[i * M + m] code bytes over row slices x[i * d + m * w .. + w);
// otherwise u32 labels[i] over whole rows (w = d <= 256).  Labels must be
// below K, and M n below 2^32 (32-bit member lists).  The member lists live
// in scratch (device words, at least kmeans_update_scratch_words(n, M, K));
// hipErrorInvalidValue when either does not hold.
size_t kmeans_update_scratch_words(int n, int M, int K);
hipError_t launch_kmeans_update(const float* x, int n, int d, int w, int M, const void* labels, bool u8,
                                int K, const uint8_t* active, bool normalize, float* out, uint32_t* scratch,
                                size_t scratch_words, hipStream_t s);

void launch_encode(const float* x, int n, int d, const float* centroids, const uint32_t* assign,
                   const float* codebooks, int M, int K, int ds, uint8_t* codes, hipStream_t s);
void launch_bias(const DevIndex& ix, float* bias, hipStream_t s);
#define TBLK_BYTES(M) (16 * (size_t)(M) + 64)
// Whether the FAST scan reads transposed blocks for this shape.
bool scan8_fast_blocks_supported(int M, int K, int ds);
// The FAST scan shapes whose per-query tables come from launch_t2_tables
// (16 codebooks of 256 codewords on transposed blocks, ds 2, 4 or 8).
bool scan8_fast_uses_tables(const DevIndex& ix);
// T2 = -2 q.cw of nq normalised queries into t2[nq][M * 256] (fp32 MFMA);
// t0 / t1 (optional) are recorded around the kernel.
void launch_t2_tables(const DevIndex& ix, const float* qn, int nq, float* t2, hipStream_t s,
                      hipEvent_t t0 = nullptr, hipEvent_t t1 = nullptr);
// Fill ix.tcodes and ix.tbias from ix.codes, ix.bias and ix.tblk_off.
void launch_tblocks(const DevIndex& ix, uint8_t* tcodes, float* tbias, hipStream_t s);
void launch_pack4(const DevIndex& ix, uint8_t* packed, hipStream_t s);
// LUT kernels for tests.
void launch_adc_tables(const float* codebooks, int M, int K, int ds, const float* r, int nr,
                       float* tables, hipStream_t s);
void launch_fastscan_test(const uint8_t* packed, int n, int M, const float* lut, float* out,
                          hipStream_t s);

// Flat exact search.
void launch_flat_norms(const float* X, int n, int d, float* norms, hipStream_t s);
size_t flat_partial_count(int nq, int n, int d, int k);
// bf16 hi/lo copy of the database for the ranking kernel (d <= 128; 0 chunks
// otherwise), in the coarse quantiser's tile-major layout.
size_t flat_pack_chunks(int n, int d);
void launch_flat_pack(const float* X, int n, int d, uint4* Xb, hipStream_t s);
// Qsq / Xnorm: squared norms (flat_norms); xmax: max ||x||; Xb: the packed
// copy (null: the fp32 ranking path for every shape); `ranked` (optional) is
// recorded between the ranking kernel and the merge.
// Queries whose kept candidates cannot be proved to hold the exact top-k are
// appended to flag_list (*overflow, zero on entry, counts them) and their
// rows are left for launch_flat_fallback.
// Qsq: the queries' squared norms; the bf16x3 ranking path (Xb) takes null
// and computes them in its merge.
void launch_flat_search(const float* Q, const float* Qsq, int nq, const float* X, const uint4* Xb,
                        const float* Xnorm, int n, int d, int k, int metric, float xmax,
                        uint64_t* partial, uint32_t* out_idx, float* out_dist,
                        unsigned int* overflow, uint32_t* flag_list, uint32_t* fbv, hipStream_t s,
                        hipEvent_t ranked = nullptr);
// The bf16x3 ranking path's fallback for the nflag queries of flag_list
// (fbv: their rescoring thresholds, written by the merge): only the slices
// whose bound does not clear the threshold are scanned exhaustively.  keys:
// scratch of nflag * flat_rank_fallback_slices(...) * k entries; 0 slices =
// the ranking path is not used for this shape.
int flat_rank_fallback_slices(int nq, int n, int d, int k);
void launch_flat_rank_fallback(const uint32_t* flag_list, int nflag, const uint32_t* fbv,
                               const uint64_t* partial, int nq, int n, int d, int k, int metric,
                               const float* Q, const float* X, uint64_t* keys, uint32_t* out_idx,
                               float* out_dist, hipStream_t s);
// The same for the first min(*nflag_dev, cap) flagged queries, the count read
// on the device (no host round trip); keys: cap * slices * k entries.
void launch_flat_rank_fallback_dev(const uint32_t* flag_list, const unsigned int* nflag_dev, int cap,
                                   const uint32_t* fbv, const uint64_t* partial, int nq, int n, int d, int k,
                                   int metric, const float* Q, const float* X, uint64_t* keys, uint32_t* out_idx,
                                   float* out_dist, hipStream_t s);
// Exhaustive exact top-k rows of the nflag queries of flag_list;
// keys: scratch of nflag * flat_fallback_slices(n, k) * k entries.
int flat_fallback_slices(int n, int k);
void launch_flat_fallback(const uint32_t* flag_list, int nflag, const float* Q, const float* X, int n, int d,
                          int k, int metric, uint64_t* keys, uint32_t* out_idx, float* out_dist,
                          hipStream_t s);

}  // namespace vgpu
