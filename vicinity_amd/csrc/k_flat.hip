// Flat exact top-k: MFMA fp32 GEMM ranking with a fused per-query candidate
// filter, then exact rescoring of the kept candidates with the reference's
// sequential arithmetic.
//
// Reference: l2_distance_squared src/distance.rs:78-83 (scalar backend
// src/simd.rs:118-121: sum (x - y)^2 in order) and cosine_distance_normalized
// src/distance.rs:104-109 (1 - dot); brute-force ground truth
// src/ivf_pq/search.rs:3376-3392.
//
// Ranking distance (metric 0): ||x||^2 - 2 q.x (||q||^2 is constant per query).
// Each block takes 64 queries and one slice of the database; every database
// tile of 64 vectors is one 64x64 MFMA tile whose scores are filtered against
// the per-query threshold into per-query LDS buffers; a full buffer is sorted
// by one wave and cut to the kept count.  The merge kernel gathers the slices,
// checks that the kept set provably contains the exact top-k (gap > 2 tau)
// and rescores it; a query that fails the check is searched exhaustively with
// the exact arithmetic.
#include "vgpu_device.h"
#include "vgpu_launch.h"

namespace vgpu {

typedef float floatx4 __attribute__((ext_vector_type(4)));

#define FL_Q 64
#define FL_N 64
#define FL_K 32
#define FL_SPLITS_MAX 64

__device__ __forceinline__ void fl_wave_sync() {
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
    __builtin_amdgcn_wave_barrier();
}

__device__ inline void fl_wave_sort(uint64_t* keys, int n) {
    const int lane = threadIdx.x & 63;
    for (int size = 2; size <= n; size <<= 1) {
        for (int stride = size >> 1; stride > 0; stride >>= 1) {
            fl_wave_sync();
            for (int t = lane; t < (n >> 1); t += 64) {
                int i = 2 * t - (t & (stride - 1));
                int j = i + stride;
                bool asc = (i & size) == 0;
                uint64_t a = keys[i], b = keys[j];
                if ((a > b) == asc) {
                    keys[i] = b;
                    keys[j] = a;
                }
            }
        }
    }
    fl_wave_sync();
}

// Sort row buffer `row` (count entries) and keep `keep`.  One wave.
__device__ inline void fl_row_flush(uint64_t* rk, uint32_t* cnt, uint32_t* thr, int cap, int keep) {
    const int lane = threadIdx.x & 63;
    int n = (int)*cnt;
    int n2 = next_pow2(n > 0 ? n : 1);
    if (n2 > cap) n2 = cap;
    for (int i = n + lane; i < n2; i += 64) rk[i] = ~0ull;
    fl_wave_sort(rk, n2);
    if (n >= keep) {
        if (lane == 0) {
            *thr = (uint32_t)(rk[keep - 1] >> 32);
            *cnt = (uint32_t)keep;
        }
    }
    fl_wave_sync();
}

__global__ void flat_norms_kernel(const float* __restrict__ X, int n, int d, float* __restrict__ out) {
    int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const float* x = X + (size_t)i * d;
    float s = 0.0f;
    for (int j = 0; j < d; j++) s += x[j] * x[j];
    out[i] = s;
}

void launch_flat_norms(const float* X, int n, int d, float* norms, hipStream_t s) {
    if (n <= 0) return;
    hipLaunchKernelGGL(flat_norms_kernel, dim3((n + 255) / 256), dim3(256), 0, s, X, n, d, norms);
}

__host__ __device__ inline int flat_keep(int k) {
    int kk = 1;
    while (kk < k + 16) kk <<= 1;
    return kk < 32 ? 32 : kk;
}

__host__ __device__ inline int flat_cap(int kk) {
    int c = 1;
    while (c < kk + FL_N) c <<= 1;
    return c;
}

__global__ __launch_bounds__(256) void flat_partial_kernel(
    const float* __restrict__ Q, const float* __restrict__ X, const float* __restrict__ Xnorm,
    int nq, int n, int d, int metric, int kk, int cap, int splits, int chunk,
    uint64_t* __restrict__ partial) {
    extern __shared__ __align__(16) char smem[];
    float (*As)[FL_K + 1] = (float (*)[FL_K + 1])smem;
    float (*Bs)[FL_K + 1] = (float (*)[FL_K + 1])(smem + FL_Q * (FL_K + 1) * 4);
    uint64_t* keys = (uint64_t*)(smem + 2 * FL_Q * (FL_K + 1) * 4);
    uint32_t* cnt = (uint32_t*)(keys + (size_t)FL_Q * cap);
    uint32_t* thr = cnt + FL_Q;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int q0 = blockIdx.x * FL_Q, s = blockIdx.y;
    const int jb = s * chunk, je = min(n, jb + chunk);
    const int wm = (wave >> 1) * 32, wn = (wave & 1) * 32;
    const int li = lane & 15, lk = lane >> 4;
    for (int r = tid; r < FL_Q; r += blockDim.x) {
        cnt[r] = 0;
        thr[r] = 0xffffffffu;
    }
    __syncthreads();
    for (int j0 = jb; j0 < je; j0 += FL_N) {
        floatx4 acc00 = {0.f, 0.f, 0.f, 0.f}, acc01 = acc00, acc10 = acc00, acc11 = acc00;
        for (int k0 = 0; k0 < d; k0 += FL_K) {
            for (int e = tid; e < FL_Q * FL_K; e += 256) {
                int r = e / FL_K, c = e % FL_K;
                int gk = k0 + c, gq = q0 + r, gx = j0 + r;
                As[r][c] = (gq < nq && gk < d) ? Q[(size_t)gq * d + gk] : 0.0f;
                Bs[r][c] = (gx < je && gk < d) ? X[(size_t)gx * d + gk] : 0.0f;
            }
            __syncthreads();
#pragma unroll
            for (int kq = 0; kq < FL_K; kq += 4) {
                float a0 = As[wm + li][kq + lk], a1 = As[wm + 16 + li][kq + lk];
                float b0 = Bs[wn + li][kq + lk], b1 = Bs[wn + 16 + li][kq + lk];
                acc00 = __builtin_amdgcn_mfma_f32_16x16x4f32(a0, b0, acc00, 0, 0, 0);
                acc01 = __builtin_amdgcn_mfma_f32_16x16x4f32(a0, b1, acc01, 0, 0, 0);
                acc10 = __builtin_amdgcn_mfma_f32_16x16x4f32(a1, b0, acc10, 0, 0, 0);
                acc11 = __builtin_amdgcn_mfma_f32_16x16x4f32(a1, b1, acc11, 0, 0, 0);
            }
            __syncthreads();
        }
        // Epilogue: filter the 16 scores of this lane into the row buffers.
#pragma unroll
        for (int t = 0; t < 4; t++) {
            const floatx4 acc = t == 0 ? acc00 : t == 1 ? acc01 : t == 2 ? acc10 : acc11;
            const int mi = t >> 1, ni = t & 1;
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const int row = wm + mi * 16 + 4 * lk + r;
                const int col = j0 + wn + ni * 16 + li;
                if (q0 + row < nq && col < je) {
                    float approx = metric == 0 ? Xnorm[col] - 2.0f * acc[r] : 1.0f - acc[r];
                    uint32_t fk = fkey(approx);
                    if (fk <= thr[row]) {
                        uint32_t slot = atomicAdd(&cnt[row], 1u);
                        keys[(size_t)row * cap + slot] = ((uint64_t)fk << 32) | (uint32_t)col;
                    }
                }
            }
        }
        __syncthreads();
        for (int row = wave; row < FL_Q; row += 4)
            if ((int)cnt[row] > cap - FL_N) fl_row_flush(keys + (size_t)row * cap, &cnt[row], &thr[row], cap, kk);
        __syncthreads();
    }
    for (int row = wave; row < FL_Q; row += 4) {
        fl_row_flush(keys + (size_t)row * cap, &cnt[row], &thr[row], cap, kk);
        if (q0 + row < nq) {
            const int have = min((int)cnt[row], kk);
            uint64_t* out = partial + ((size_t)(q0 + row) * splits + s) * kk;
            for (int i = lane; i < kk; i += 64) out[i] = i < have ? keys[(size_t)row * cap + i] : ~0ull;
        }
    }
}

#define FL_BUF 1024
#define FL_ROUND 512

__device__ inline float flat_exact(const float* q, const float* x, int d, int metric) {
    if (metric == 0) {
        float s = 0.0f;
        for (int j = 0; j < d; j++) {
            float t = q[j] - x[j];
            s += t * t;
        }
        return s;
    }
    return 1.0f - seq_dot(q, x, d);
}

__global__ __launch_bounds__(256) void flat_merge_kernel(
    const uint64_t* __restrict__ partial, int splits, int kk, const float* __restrict__ Q,
    const float* __restrict__ Qsq, const float* __restrict__ X, int nq, int n, int d, int k,
    int metric, float xmax, uint32_t* __restrict__ out_idx, float* __restrict__ out_dist,
    unsigned int* overflow) {
    __shared__ uint64_t keys[FL_BUF];
    __shared__ uint32_t pay[FL_BUF];
    __shared__ uint32_t misc[4];
    const int q = blockIdx.x, tid = threadIdx.x;
    if (q >= nq) return;
    const float* qv = Q + (size_t)q * d;
    const int tot = splits * kk;
    const int n2 = next_pow2(tot);
    for (int i = tid; i < n2; i += blockDim.x) {
        keys[i] = i < tot ? partial[(size_t)q * tot + i] : ~0ull;
        pay[i] = 0;
    }
    block_bitonic_sort(keys, pay, n2);
    if (tid == 0) {
        int have = 0;
        while (have < kk && keys[have] != ~0ull) have++;
        uint32_t fail = 0;
        if (n > have && have >= k) {
            const float u = 5.9604645e-08f;
            const float qmax = sqrtf(Qsq[q]) * 1.0001f + 1e-30f;
            float tau = metric == 0 ? 4.0f * (float)(d + 8) * u * (qmax + xmax) * (qmax + xmax)
                                    : 4.0f * (float)(d + 8) * u * (1.0f + qmax * xmax);
            float gap = key_dist(keys[have - 1]) - key_dist(keys[k - 1]);
            if (!(gap > 2.0f * tau)) fail = 1;
        }
        misc[0] = (uint32_t)have;
        misc[1] = fail;
        if (fail) atomicAdd(overflow, 1u);
    }
    __syncthreads();
    const int have = (int)misc[0];
    if (!misc[1]) {
        for (int i = tid; i < n2; i += blockDim.x) {
            if (i < have) {
                uint32_t idx = (uint32_t)keys[i];
                keys[i] = cand_key(flat_exact(qv, X + (size_t)idx * d, d, metric), idx);
            } else {
                keys[i] = ~0ull;
            }
        }
        block_bitonic_sort(keys, pay, n2);
    } else {
        // Exhaustive exact scan with a threshold-filtered LDS buffer.
        if (tid == 0) {
            misc[2] = 0;
            misc[3] = 0xffffffffu;
        }
        __syncthreads();
        for (int base = 0; base < n; base += FL_ROUND) {
            if ((int)misc[2] > FL_BUF - FL_ROUND) {
                int m = (int)misc[2];
                int m2 = next_pow2(m);
                for (int i = m + tid; i < m2; i += blockDim.x) keys[i] = ~0ull;
                block_bitonic_sort(keys, pay, m2);
                if (tid == 0 && m >= k) {
                    misc[3] = (uint32_t)(keys[k - 1] >> 32);
                    misc[2] = (uint32_t)k;
                }
                __syncthreads();
            }
            const uint32_t th = misc[3];
            for (int u = 0; u < FL_ROUND / 256; u++) {
                int j = base + u * 256 + tid;
                bool take = false;
                uint64_t key = 0;
                if (j < n) {
                    float dist = flat_exact(qv, X + (size_t)j * d, d, metric);
                    key = cand_key(dist, (uint32_t)j);
                    take = (uint32_t)(key >> 32) <= th;
                }
                int slot = wave_append_slot(take, &misc[2]);
                if (take) keys[slot] = key;
            }
            __syncthreads();
        }
        int m = (int)misc[2];
        int m2 = next_pow2(m > 0 ? m : 1);
        for (int i = m + tid; i < m2; i += blockDim.x) keys[i] = ~0ull;
        block_bitonic_sort(keys, pay, m2);
    }
    for (int j = tid; j < k; j += blockDim.x) {
        size_t o = (size_t)q * k + j;
        uint64_t key = keys[j];
        if (j < n && key != ~0ull) {
            out_idx[o] = (uint32_t)key;
            out_dist[o] = key_dist(key);
        } else {
            out_idx[o] = 0xffffffffu;
            out_dist[o] = __int_as_float(0x7f800000);
        }
    }
}

// Database slices per query block: enough blocks to fill the GPU, slices of
// at least 4 tiles, and splits * kk merge entries within the merge buffer.
static int flat_splits(int nq, int n, int kk) {
    int qb = (nq + FL_Q - 1) / FL_Q;
    int sp = 1;
    while (sp < FL_SPLITS_MAX && qb * sp < 2048 && 2 * sp * kk <= FL_BUF &&
           (n + sp * 2 - 1) / (sp * 2) >= 4 * FL_N)
        sp <<= 1;
    return sp;
}

size_t flat_partial_count(int nq, int n, int k) {
    return (size_t)nq * flat_splits(nq, n, flat_keep(k)) * flat_keep(k);
}

void launch_flat_search(const float* Q, const float* Qsq, int nq, const float* X,
                        const float* Xnorm, int n, int d, int k, int metric, float xmax,
                        uint64_t* partial, uint32_t* out_idx, float* out_dist,
                        unsigned int* overflow, hipStream_t s) {
    if (nq <= 0) return;
    const int kk = flat_keep(k), cap = flat_cap(kk), sp = flat_splits(nq, n, kk);
    const int chunk = (((n + sp - 1) / sp) + FL_N - 1) / FL_N * FL_N;
    size_t lds = 2 * FL_Q * (FL_K + 1) * 4 + (size_t)FL_Q * cap * 8 + 2 * FL_Q * 4;
    ensure_dyn_lds((const void*)flat_partial_kernel, lds);
    dim3 grid((nq + FL_Q - 1) / FL_Q, sp);
    hipLaunchKernelGGL(flat_partial_kernel, grid, dim3(256), lds, s, Q, X, Xnorm, nq, n, d, metric, kk,
                       cap, sp, chunk, partial);
    hipLaunchKernelGGL(flat_merge_kernel, dim3(nq), dim3(256), 0, s, partial, sp, kk, Q, Qsq, X, nq, n,
                       d, k, metric, xmax, out_idx, out_dist, overflow);
}

}  // namespace vgpu
