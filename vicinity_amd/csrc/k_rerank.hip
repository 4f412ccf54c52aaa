// Exact rerank of the approximate pool and the final id mapping / padding.
//
// Reference: search_reranked src/ivf_pq/search.rs:1117-1158 (exact
// cosine_distance_normalized 1 - dot(q, v) over the stored normalised vector,
// src/distance.rs:104-109, then finish_top_k_by_distance :64-75);
// search :1087-1093 (insertion index -> doc id); batch padding
// src/python.rs:778-785 (MISSING_LABEL -1, MISSING_DISTANCE +inf).
#include "vgpu_device.h"
#include "vgpu_launch.h"

namespace vgpu {

// One workgroup per query; the pool's keys, a payload row (next_pow2(pool)
// of each; pool <= RERANK_MAX) and the query in dynamic LDS.  Each thread
// streams its candidate's row 32 floats at a time (seq_dot_stream: the same
// sequential sum).
__global__ __launch_bounds__(256) void rerank_kernel(const float* __restrict__ vectors, int d,
                                                     const float* __restrict__ qn, int nq,
                                                     const uint32_t* __restrict__ pool_vidx,
                                                     int pool, int k, uint32_t* __restrict__ out_vidx,
                                                     float* __restrict__ out_dist) {
    extern __shared__ __align__(16) uint64_t keys[];
    const int q = blockIdx.x;
    if (q >= nq) return;
    const int n2 = next_pow2(pool);
    uint32_t* pay = reinterpret_cast<uint32_t*>(keys + n2);
    float* qs = reinterpret_cast<float*>(pay + n2);  // [d]
    for (int j = threadIdx.x; j < d; j += blockDim.x) qs[j] = qn[(size_t)q * d + j];
    __syncthreads();
    for (int t = threadIdx.x; t < n2; t += blockDim.x) {
        uint64_t key = ~0ull;
        if (t < pool) {
            uint32_t v = pool_vidx[(size_t)q * pool + t];
            if (v != 0xffffffffu) key = cand_key(1.0f - seq_dot_stream(qs, vectors + (size_t)v * d, d), v);
        }
        keys[t] = key;
        pay[t] = 0;
    }
    block_bitonic_sort(keys, pay, n2);
    for (int j = threadIdx.x; j < k; j += blockDim.x) {
        uint64_t key = j < pool ? keys[j] : ~0ull;
        size_t o = (size_t)q * k + j;
        if (key != ~0ull) {
            out_vidx[o] = (uint32_t)key;
            out_dist[o] = key_dist(key);
        } else {
            out_vidx[o] = 0xffffffffu;
            out_dist[o] = __int_as_float(0x7f800000);
        }
    }
}

static size_t rerank_lds(int pool, int d) {
    size_t n2 = 1;
    while (n2 < (size_t)pool) n2 <<= 1;
    return n2 * (sizeof(uint64_t) + sizeof(uint32_t)) + (size_t)d * sizeof(float);
}

void launch_rerank(const DevIndex& ix, const float* qn, int nq, const uint32_t* pool_vidx,
                   int pool, int k, uint32_t* out_vidx, float* out_dist, hipStream_t s) {
    launch_rerank_vectors(ix.vectors, ix.d, qn, nq, pool_vidx, pool, k, out_vidx, out_dist, s);
}

void launch_rerank_vectors(const float* vectors, int d, const float* qn, int nq, const uint32_t* pool_rows,
                           int pool, int k, uint32_t* out_rows, float* out_dist, hipStream_t s) {
    if (nq <= 0) return;
    const size_t lds = rerank_lds(pool, d);
    ensure_dyn_lds((const void*)rerank_kernel, lds);
    hipLaunchKernelGGL(rerank_kernel, dim3(nq), dim3(256), lds, s, vectors, d, qn, nq, pool_rows, pool, k,
                       out_rows, out_dist);
}

__global__ void finalize_kernel(const uint32_t* __restrict__ vidx, const float* __restrict__ dist,
                                const uint32_t* __restrict__ doc_ids, int nq, int kin, int k,
                                int64_t* __restrict__ out_ids, float* __restrict__ out_dists) {
    const size_t e = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (e >= (size_t)nq * k) return;
    const size_t q = e / k, j = e % k;
    uint32_t v = j < (size_t)kin ? vidx[q * kin + j] : 0xffffffffu;
    if (v != 0xffffffffu) {
        out_ids[e] = (int64_t)(doc_ids ? doc_ids[v] : v);
        out_dists[e] = dist[q * kin + j];
    } else {
        out_ids[e] = -1;
        out_dists[e] = __int_as_float(0x7f800000);
    }
}

void launch_finalize(const uint32_t* vidx, const float* dist, const uint32_t* doc_ids, int nq,
                     int kin, int k, int64_t* out_ids, float* out_dists, hipStream_t s) {
    size_t total = (size_t)nq * k;
    if (total == 0) return;
    hipLaunchKernelGGL(finalize_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, s, vidx,
                       dist, doc_ids, nq, kin, k, out_ids, out_dists);
}

// End of a search chunk, FINISH_Q queries per workgroup: map insertion indices to
// doc ids with (-1, +inf) padding (python.rs:778-785; skipped when vidx is null:
// the scan wrote the final rows, and each workgroup then takes the statistics
// of 128 queries), add the statistics rows
// into the counters (every FINISH_STATS-th workgroup adds 128 queries' rows,
// one atomic per counter; counters sit COUNTER_STRIDE words apart), and clear
// the two flag-list lengths for the next chunk (both lists were consumed by
// earlier launches).
#define FINISH_Q 16
#define FINISH_STATS 8  // workgroups per statistics row block (128 queries)
static_assert(FINISH_Q * FINISH_STATS == 128, "two queries per lane");

__global__ __launch_bounds__(256) void finish_kernel(
    const uint32_t* __restrict__ vidx, const float* __restrict__ dist,
    const uint32_t* __restrict__ doc_ids, int nq, int kin, int k, int64_t* __restrict__ out_ids,
    float* __restrict__ out_dists, const uint32_t* __restrict__ qstat,
    unsigned long long* __restrict__ counters, uint32_t* flag_count, uint32_t* cflag_count,
    const uint32_t* __restrict__ qbad) {
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const bool map = vidx != nullptr;
    const int q0 = blockIdx.x * (map ? FINISH_Q : FINISH_Q * FINISH_STATS);
    const int nqb = min(FINISH_Q, nq - q0);
    // wave w takes rows w, w + 4, ...; a lane takes columns lane, lane + 64, ...
    constexpr int U = 8;  // outputs per lane whose loads are in flight together
    constexpr int RW = FINISH_Q / (VGPU_BLOCK / 64);  // rows per wave
    for (int c0 = 0; map && c0 < k; c0 += 64 * (U / RW)) {
        uint32_t v[U], id[U];
        float dv[U];
#pragma unroll
        for (int u = 0; u < U; u++) {
            const int r = wave + (VGPU_BLOCK / 64) * (u % RW), j = c0 + lane + 64 * (u / RW);
            v[u] = r < nqb && j < k && j < kin ? vidx[(size_t)(q0 + r) * kin + j] : 0xffffffffu;
            if (qbad && r < nqb && qbad[q0 + r]) v[u] = 0xffffffffu;  // non-finite query
        }
#pragma unroll
        for (int u = 0; u < U; u++) {
            const int r = wave + (VGPU_BLOCK / 64) * (u % RW), j = c0 + lane + 64 * (u / RW);
            const bool ok = v[u] != 0xffffffffu;
            id[u] = ok && doc_ids ? doc_ids[v[u]] : v[u];
            dv[u] = ok ? dist[(size_t)(q0 + r) * kin + j] : __int_as_float(0x7f800000);
        }
#pragma unroll
        for (int u = 0; u < U; u++) {
            const int r = wave + (VGPU_BLOCK / 64) * (u % RW), j = c0 + lane + 64 * (u / RW);
            if (r < nqb && j < k) {
                const size_t o = (size_t)(q0 + r) * k + j;
                out_ids[o] = v[u] != 0xffffffffu ? (int64_t)id[u] : (int64_t)-1;
                out_dists[o] = dv[u];
            }
        }
    }
    // rows written by the scan: a non-finite query's row becomes padding
    if (!map && qbad && wave < 2) {
        const int r = wave * 64 + lane;
        uint64_t m = __ballot(q0 + r < nq && qbad[q0 + r] != 0u);
        while (m) {
            const int b = __ffsll((unsigned long long)m) - 1;
            m &= m - 1;
            const size_t row = (size_t)(q0 + wave * 64 + b) * k;
            for (int j = lane; j < k; j += 64) {
                out_ids[row + j] = -1;
                out_dists[row + j] = __int_as_float(0x7f800000);
            }
        }
    }
    // statistics: every FINISH_STATS-th workgroup adds 128 queries' rows
    if (qstat && tid < 64 && (!map || blockIdx.x % FINISH_STATS == 0)) {
        uint32_t c[NUM_SCAN_COUNTERS] = {0, 0, 0, 0, 0, 0};
#pragma unroll
        for (int h = 0; h < 2; h++) {
            const int qq = q0 + h * 64 + lane;
            if (qq < nq) {
                const uint32_t* st = qstat + (size_t)qq * QSTAT_WORDS;
                c[0] += st[0];              // entries scanned
                c[1] += st[3] & 1u;         // fallbacks
                c[2] += st[1];              // flushes
                c[3] += st[2];              // appends
                c[4] += (st[3] >> 1) & 1u;  // fallbacks from ties
                c[5] += (st[3] >> 2) & 1u;  // second passes
            }
        }
#pragma unroll
        for (int i = 0; i < NUM_SCAN_COUNTERS; i++) {
            unsigned long long v = c[i];
            for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
            if (lane == 0 && v) atomicAdd(&counters[i * COUNTER_STRIDE], v);
        }
    }
    if (blockIdx.x == 0 && tid == 0) {
        if (flag_count) *flag_count = 0u;
        if (cflag_count) {
            counters[NUM_SCAN_COUNTERS * COUNTER_STRIDE] += *cflag_count;  // exact coarse fallbacks
            *cflag_count = 0u;
        }
    }
}

void launch_finish(const uint32_t* vidx, const float* dist, const uint32_t* doc_ids, int nq, int kin,
                   int k, int64_t* out_ids, float* out_dists, const uint32_t* qstat,
                   unsigned long long* counters, uint32_t* flag_count, uint32_t* cflag_count,
                   hipStream_t s, const uint32_t* qbad) {
    if (nq <= 0) return;
    const int per = vidx ? FINISH_Q : FINISH_Q * FINISH_STATS;
    hipLaunchKernelGGL(finish_kernel, dim3((nq + per - 1) / per), dim3(VGPU_BLOCK), 0, s, vidx,
                       dist, doc_ids, nq, kin, k, out_ids, out_dists, qstat, counters, flag_count,
                       cflag_count, qbad);
}

// Clear n 64-bit words (the per-call scalars) with a kernel, not a
// memset, so a captured stream records a kernel node.
__global__ void zero_words_kernel(unsigned long long* __restrict__ p, size_t n) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) p[i] = 0ull;
}

void launch_zero_words(unsigned long long* p, size_t n, hipStream_t s) {
    if (n == 0) return;
    hipLaunchKernelGGL(zero_words_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, p, n);
}

}  // namespace vgpu
