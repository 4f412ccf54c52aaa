// Query normalisation and the coarse quantiser: an MFMA fp32 GEMM of queries
// against centroids, then per-query selection of the nprobe lists with exact
// rescoring of every list whose MFMA score lies inside the rounding margin.
//
// Reference: normalize_query src/ivf_pq/search.rs:55-62; find_nearest_centroids
// search.rs:1602-1617 with cosine_distance_normalized src/distance.rs:104-109
// (score 1 - dot(q, c), nprobe smallest, ascending).
#include "vgpu_device.h"
#include "vgpu_launch.h"

namespace vgpu {

typedef float floatx4 __attribute__((ext_vector_type(4)));

// One thread per row: s = sum x^2 in order, norm = sqrt(s), x / norm when
// norm > 1e-10 (search.rs:55-62; divide and sqrt are correctly rounded).
// norms[i] receives an upper bound of ||out_i|| used by the error margins.
__global__ void normalize_kernel(const float* __restrict__ x, float* __restrict__ out,
                                 float* __restrict__ norms, int n, int d) {
    int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const float* xi = x + (size_t)i * d;
    float* oi = out + (size_t)i * d;
    float s = 0.0f;
    for (int j = 0; j < d; j++) s += xi[j] * xi[j];
    float nrm = sqrtf(s);
    if (nrm > 1e-10f) {
        for (int j = 0; j < d; j++) oi[j] = xi[j] / nrm;
        if (norms) norms[i] = 1.0001f;
    } else {
        for (int j = 0; j < d; j++) oi[j] = xi[j];
        if (norms) norms[i] = nrm * 1.0001f;
    }
}

void launch_normalize(const float* x, float* out, float* norms, int n, int d, hipStream_t s) {
    if (n <= 0) return;
    hipLaunchKernelGGL(normalize_kernel, dim3((n + 255) / 256), dim3(256), 0, s, x, out, norms, n, d);
}

// ---- coarse GEMM --------------------------------------------------------
// D[q][c] = sum_k Q[q][k] * C[c][k] with v_mfma_f32_16x16x4_f32.
// Block tile 64 (queries) x 64 (centroids), 4 waves each own a 32x32 quarter
// as 2x2 MFMA tiles.  Operand layout of 16x16x4 f32 (wave64): A[i][k] comes
// from lane i + 16k, B[k][j] from lane j + 16k, D[i][j] lands in lane
// j + 16*(i/4), element i%4.
#define CT_M 64
#define CT_N 64
#define CT_K 32

__global__ __launch_bounds__(256) void coarse_dots_kernel(const float* __restrict__ Q,
                                                          const float* __restrict__ C,
                                                          float* __restrict__ D, int nq, int L,
                                                          int d) {
    __shared__ float As[CT_M][CT_K + 1];
    __shared__ float Bs[CT_N][CT_K + 1];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int row0 = blockIdx.y * CT_M, col0 = blockIdx.x * CT_N;
    const int wm = (wave >> 1) * 32, wn = (wave & 1) * 32;
    floatx4 acc00 = {0.f, 0.f, 0.f, 0.f}, acc01 = acc00, acc10 = acc00, acc11 = acc00;
    const int li = lane & 15, lk = lane >> 4;
    for (int k0 = 0; k0 < d; k0 += CT_K) {
        for (int e = tid; e < CT_M * CT_K; e += 256) {
            int r = e / CT_K, c = e % CT_K;
            int gk = k0 + c;
            int gr = row0 + r, gc = col0 + r;
            As[r][c] = (gr < nq && gk < d) ? Q[(size_t)gr * d + gk] : 0.0f;
            Bs[r][c] = (gc < L && gk < d) ? C[(size_t)gc * d + gk] : 0.0f;
        }
        __syncthreads();
#pragma unroll
        for (int kk = 0; kk < CT_K; kk += 4) {
            float a0 = As[wm + li][kk + lk];
            float a1 = As[wm + 16 + li][kk + lk];
            float b0 = Bs[wn + li][kk + lk];
            float b1 = Bs[wn + 16 + li][kk + lk];
            acc00 = __builtin_amdgcn_mfma_f32_16x16x4f32(a0, b0, acc00, 0, 0, 0);
            acc01 = __builtin_amdgcn_mfma_f32_16x16x4f32(a0, b1, acc01, 0, 0, 0);
            acc10 = __builtin_amdgcn_mfma_f32_16x16x4f32(a1, b0, acc10, 0, 0, 0);
            acc11 = __builtin_amdgcn_mfma_f32_16x16x4f32(a1, b1, acc11, 0, 0, 0);
        }
        __syncthreads();
    }
    const int rbase = row0 + wm + 4 * lk;
    const int cbase = col0 + wn + li;
#pragma unroll
    for (int r = 0; r < 4; r++) {
        int r0 = rbase + r, r1 = rbase + 16 + r;
        if (r0 < nq) {
            if (cbase < L) D[(size_t)r0 * L + cbase] = acc00[r];
            if (cbase + 16 < L) D[(size_t)r0 * L + cbase + 16] = acc01[r];
        }
        if (r1 < nq) {
            if (cbase < L) D[(size_t)r1 * L + cbase] = acc10[r];
            if (cbase + 16 < L) D[(size_t)r1 * L + cbase + 16] = acc11[r];
        }
    }
}

void launch_coarse_dots(const float* Q, const float* C, float* D, int nq, int L, int d,
                        hipStream_t s) {
    if (nq <= 0 || L <= 0) return;
    dim3 grid((L + CT_N - 1) / CT_N, (nq + CT_M - 1) / CT_M);
    hipLaunchKernelGGL(coarse_dots_kernel, grid, dim3(256), 0, s, Q, C, D, nq, L, d);
}

// ---- probe selection ----------------------------------------------------
#define SEL_CAP 1024

// Error bound of the MFMA score against the sequential one: both are within
// (d + 2) u sum|q_j c_j| <= (d + 2) u ||q|| ||c|| of the real dot product,
// plus the rounding of 1 - dot; doubled for safety.
__device__ __forceinline__ float coarse_tau(int d, float qn, float cmax) {
    const float u = 5.9604645e-08f;
    return 2.0f * ((2.0f * (float)d + 8.0f) * u * qn * cmax + 4.0f * u * (1.0f + qn * cmax)) +
           1e-30f;
}

__global__ __launch_bounds__(256) void coarse_select_kernel(
    float* __restrict__ D, const float* __restrict__ qn, const float* __restrict__ qnorm,
    const float* __restrict__ C, int nq, int L, int d, int P, float cmax,
    uint32_t* __restrict__ probe, unsigned int* overflow) {
    __shared__ RadixScratch rs;
    __shared__ uint64_t keys[SEL_CAP];
    __shared__ uint32_t pay[SEL_CAP];
    __shared__ uint32_t cnt;
    const int tid = threadIdx.x;
    const int q = blockIdx.x;
    if (q >= nq) return;
    float* row = D + (size_t)q * L;
    const float* qv = qn + (size_t)q * d;
    const int Pe = P < L ? P : L;

    // Rank Pe-1 of the approximate scores 1 - dot.
    auto akey = [&](int i) -> uint32_t { return fkey(1.0f - row[i]); };
    uint32_t T = block_radix_select<uint32_t>(akey, L, (uint32_t)(Pe - 1), &rs);
    float W = fkey_to_float(T) + 2.0f * coarse_tau(d, qnorm[q], cmax);
    uint32_t WK = fkey(W);
    if (WK < T) WK = T;  // keeps the Pe smallest inside the window for any input

    if (tid == 0) cnt = 0;
    __syncthreads();
    for (int i = tid; i < L; i += blockDim.x) {
        if (akey(i) <= WK) {
            uint32_t slot = atomicAdd(&cnt, 1u);
            if (slot < SEL_CAP) keys[slot] = (uint64_t)i;
        }
    }
    __syncthreads();
    const uint32_t cn = cnt;
    if (cn <= SEL_CAP) {
        // Exact 1 - dot in the reference's order for every margin candidate.
        for (uint32_t t = tid; t < cn; t += blockDim.x) {
            uint32_t c = (uint32_t)keys[t];
            float ex = 1.0f - seq_dot(qv, C + (size_t)c * d, d);
            keys[t] = cand_key(ex, c);
            pay[t] = c;
        }
        int n2 = next_pow2((int)cn);
        for (int t = (int)cn + tid; t < n2; t += blockDim.x) {
            keys[t] = ~0ull;
            pay[t] = 0xffffffffu;
        }
        block_bitonic_sort(keys, pay, n2);
        for (int p = tid; p < Pe; p += blockDim.x) probe[(size_t)q * P + p] = pay[p];
        return;
    }
    // Overflow (degenerate inputs such as a zero query): exact scores of all
    // margin candidates replace the row (+inf elsewhere), then an exact
    // 64-bit radix select.  Each thread rereads only the entries it wrote.
    if (tid == 0) atomicAdd(overflow, 1u);
    for (int i = tid; i < L; i += blockDim.x) {
        bool cand = akey(i) <= WK;
        row[i] = cand ? 1.0f - seq_dot(qv, C + (size_t)i * d, d) : __int_as_float(0x7f800000);
    }
    auto ekey = [&](int i) -> uint64_t { return cand_key(row[i], (uint32_t)i); };
    uint64_t K64 = block_radix_select<uint64_t>(ekey, L, (uint32_t)(Pe - 1), &rs);
    if (tid == 0) cnt = 0;
    __syncthreads();
    for (int i = tid; i < L; i += blockDim.x) {
        uint64_t k = ekey(i);
        if (k <= K64) {
            uint32_t slot = atomicAdd(&cnt, 1u);
            if (slot < SEL_CAP) {
                keys[slot] = k;
                pay[slot] = (uint32_t)i;
            }
        }
    }
    __syncthreads();
    int n2 = next_pow2(Pe);
    for (int t = Pe + tid; t < n2; t += blockDim.x) {
        keys[t] = ~0ull;
        pay[t] = 0xffffffffu;
    }
    block_bitonic_sort(keys, pay, n2);
    for (int p = tid; p < Pe; p += blockDim.x) probe[(size_t)q * P + p] = pay[p];
}

void launch_coarse_select(float* D, const float* qn, const float* qnorm, const float* C, int nq,
                          int L, int d, int P, float cmax, uint32_t* probe,
                          unsigned int* overflow, hipStream_t s) {
    if (nq <= 0) return;
    hipLaunchKernelGGL(coarse_select_kernel, dim3(nq), dim3(256), 0, s, D, qn, qnorm, C, nq, L, d,
                       P, cmax, probe, overflow);
}

}  // namespace vgpu
