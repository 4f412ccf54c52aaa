// Query normalisation and the coarse quantiser: an MFMA fp32 GEMM of queries
// against centroids, then per-query selection of the nprobe lists with exact
// rescoring of every list whose MFMA score lies inside the rounding margin.
//
// Reference: normalize_query src/ivf_pq/search.rs:55-62; find_nearest_centroids
// search.rs:1602-1617 with cosine_distance_normalized src/distance.rs:104-109
// (score 1 - dot(q, c), nprobe smallest, ascending).
#include "vgpu_device.h"
#include "vgpu_bounds.h"
#include "vgpu_launch.h"

namespace vgpu {

typedef float floatx4 __attribute__((ext_vector_type(4)));

// Sixteen rows per workgroup, staged through LDS (row stride d + 1 keeps the
// sequential per-row reads free of bank conflicts): s = sum x^2 in order by
// one lane per row, norm = sqrt(s), then every element x / norm when
// norm > 1e-10 (search.rs:55-62; divide and sqrt are correctly rounded).
// norms[i] receives an upper bound of ||out_i|| used by the error margins.
// A row holding a NaN or an infinity is searched as the zero vector (every
// later kernel sees finite values), marked in qbad[i] (when given) and
// counted in *nbad, so the host reports it and its result row is padding.
#define NR_ROWS 16

__global__ __launch_bounds__(256) void normalize_kernel(const float* __restrict__ x,
                                                        float* __restrict__ out,
                                                        float* __restrict__ norms, int n, int d,
                                                        uint32_t* __restrict__ qbad,
                                                        unsigned int* __restrict__ nbad) {
    extern __shared__ float srow[];  // [NR_ROWS][d + 1]
    __shared__ float snorm[NR_ROWS];
    const int tid = threadIdx.x;
    const int r0 = blockIdx.x * NR_ROWS;
    const int rows = min(NR_ROWS, n - r0);
    const int st = d + 1;
    const float* src = x + (size_t)r0 * d;
    for (int e = tid; e < rows * d; e += VGPU_BLOCK) srow[(e / d) * st + e % d] = src[e];
    __syncthreads();
    if (tid < rows) {
        float* xr = srow + tid * st;
        if (row_nonfinite(xr, d)) {
            for (int j = 0; j < d; j++) xr[j] = 0.0f;
            if (nbad) atomicAdd(nbad, 1u);
            if (qbad) qbad[r0 + tid] = 1u;
        } else if (qbad) {
            qbad[r0 + tid] = 0u;
        }
        float s = 0.0f;
        for (int j = 0; j < d; j++) s = __fadd_rn(s, __fmul_rn(xr[j], xr[j]));
        const float nrm = sqrtf(s);
        snorm[tid] = nrm;
        if (norms) norms[r0 + tid] = nrm > 1e-10f ? 1.0001f : nrm * 1.0001f;
    }
    __syncthreads();
    float* dst = out + (size_t)r0 * d;
    for (int e = tid; e < rows * d; e += VGPU_BLOCK) {
        const int r = e / d;
        const float v = srow[r * st + e % d], nrm = snorm[r];
        dst[e] = nrm > 1e-10f ? v / nrm : v;
    }
}

void launch_normalize(const float* x, float* out, float* norms, int n, int d, hipStream_t s,
                      uint32_t* qbad, unsigned int* nbad) {
    if (n <= 0) return;
    const size_t lds = (size_t)NR_ROWS * (d + 1) * sizeof(float);
    ensure_dyn_lds((const void*)normalize_kernel, lds);
    hipLaunchKernelGGL(normalize_kernel, dim3((n + NR_ROWS - 1) / NR_ROWS), dim3(VGPU_BLOCK), lds, s,
                       x, out, norms, n, d, qbad, nbad);
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

// Exact ordering of the window candidates keys[0..cn) (list indices on entry):
// rescore 1 - dot in the reference's sequential order, sort by (score, list),
// write the first Pe.  cn <= SEL_CAP.  All threads call it.
// qs: LDS scratch of at least d floats.
__device__ inline void select_window_exact(uint64_t* keys, uint32_t cn, const float* qv, float* qs,
                                           const float* __restrict__ C, int d, int Pe, int P,
                                           int q, uint32_t* __restrict__ probe) {
    const int tid = threadIdx.x, lane = tid & 63;
    for (int j = tid; j < d; j += VGPU_BLOCK) qs[j] = qv[j];
    __syncthreads();
    for (uint32_t t = tid; t < cn; t += VGPU_BLOCK) {
        const uint32_t c = (uint32_t)keys[t];
        keys[t] = cand_key(1.0f - seq_dot_stream(qs, C + (size_t)c * d, d), c);
    }
    __syncthreads();
    if (cn <= 64) {  // one wave, keys in registers
        if (tid < 64) {
            uint64_t k1[1] = {(uint32_t)lane < cn ? keys[lane] : ~0ull};
            wave_sort_regs<1>(k1);
            if (lane < Pe) probe[(size_t)q * P + lane] = (uint32_t)k1[0];
        }
        return;
    }
    if (cn <= 256) {
        if (tid < 64) {
            uint64_t k4[4];
#pragma unroll
            for (int e = 0; e < 4; e++) k4[e] = (uint32_t)(e * 64 + lane) < cn ? keys[e * 64 + lane] : ~0ull;
            wave_sort_regs<4>(k4);
#pragma unroll
            for (int e = 0; e < 4; e++)
                if (e * 64 + lane < Pe) probe[(size_t)q * P + e * 64 + lane] = (uint32_t)k4[e];
        }
        return;
    }
    const int n2 = next_pow2((int)cn);
    for (int t = (int)cn + tid; t < n2; t += VGPU_BLOCK) keys[t] = ~0ull;
    block_bitonic_sort_keys(keys, n2);
    for (int p = tid; p < Pe; p += VGPU_BLOCK) probe[(size_t)q * P + p] = (uint32_t)keys[p];
}

// Probe selection with the scores of one query held in registers (EPT per
// thread, L <= 256 * EPT), one read of the score row.  The Pe-th smallest of
// the 256 per-thread minima, T, bounds the Pe-th smallest score from above (Pe
// distinct threads hold a score <= T), so every list whose exact score can be
// among the Pe smallest has approximate score <= T + 2 tau.  Those are rescored
// exactly and sorted.  Pe <= 256.
// row: the query's L dot products (global or LDS; overwritten for degenerate
// windows); qv: the normalised query.
template <int EPT>
__device__ void select_block_query(float* row, const float* __restrict__ qv, float qnorm_q,
                                   const float* __restrict__ C, int q, int L, int d, int P,
                                   float cmax, uint32_t* __restrict__ probe, unsigned int* overflow) {
    __shared__ RadixScratch rs;
    __shared__ uint64_t keys[SEL_CAP];
    __shared__ uint32_t pay[SEL_CAP];
    __shared__ uint32_t mins[VGPU_BLOCK];
    __shared__ uint32_t cnt, tsel;
    const int tid = threadIdx.x, lane = tid & 63;
    const int Pe = P < L ? P : L;

    uint32_t fk[EPT];
    uint32_t mn = 0xffffffffu;
    float sv[EPT];  // unconditional loads (clamped index) so all EPT are in flight together
#pragma unroll
    for (int e = 0; e < EPT; e++) {
        const int i = e * VGPU_BLOCK + tid;
        sv[e] = row[i < L ? i : L - 1];
    }
#pragma unroll
    for (int e = 0; e < EPT; e++) {
        const int i = e * VGPU_BLOCK + tid;
        fk[e] = i < L ? fkey(1.0f - sv[e]) : 0xffffffffu;
        mn = fk[e] < mn ? fk[e] : mn;
    }
    mins[tid] = mn;
    if (tid == 0) cnt = 0;
    __syncthreads();
    if (tid < 64) {
        uint64_t k4[4];
#pragma unroll
        for (int e = 0; e < 4; e++) k4[e] = mins[e * 64 + lane];
        wave_sort_regs<4>(k4);
        const int idx = Pe - 1;
        uint64_t v = k4[0];
#pragma unroll
        for (int e = 1; e < 4; e++) v = (idx >> 6) == e ? k4[e] : v;
        v = __shfl(v, idx & 63, 64);
        if (lane == 0) tsel = (uint32_t)v;
    }
    __syncthreads();
    const uint32_t T = tsel;
    const float W = fkey_to_float(T) + 2.0f * coarse_tau(d, qnorm_q, cmax);
    uint32_t WK = fkey(W);
    WK = WK < 0xfffffffeu ? WK + 1u : 0xffffffffu;  // one ulp to spare
    if (WK < T) WK = T;
#pragma unroll
    for (int e = 0; e < EPT; e++) {
        const int i = e * VGPU_BLOCK + tid;
        const bool take = i < L && fk[e] <= WK;
        const int slot = wave_append_slot(take, &cnt);
        if (take && slot < SEL_CAP) keys[slot] = (uint64_t)i;
    }
    __syncthreads();
    const uint32_t cn = cnt;
    if (cn <= SEL_CAP) {  // pay doubles as the query's LDS copy (d <= SEL_CAP)
        select_window_exact(keys, cn, qv, reinterpret_cast<float*>(pay), C, d, Pe, P, q, probe);
        return;
    }
    // Overflow (degenerate inputs such as a zero query): exact scores of all
    // window candidates replace the row (+inf elsewhere), then an exact
    // 64-bit radix select.  Each thread rereads only the entries it wrote.
    if (tid == 0) atomicAdd(overflow, 1u);
#pragma unroll
    for (int e = 0; e < EPT; e++) {
        const int i = e * VGPU_BLOCK + tid;
        if (i < L) row[i] = fk[e] <= WK ? 1.0f - seq_dot(qv, C + (size_t)i * d, d)
                                        : __int_as_float(0x7f800000);
    }
    auto ekey = [&](int i) -> uint64_t { return cand_key(row[i], (uint32_t)i); };
    const uint64_t K64 = block_radix_select<uint64_t>(ekey, L, (uint32_t)(Pe - 1), &rs);
    if (tid == 0) cnt = 0;
    __syncthreads();
    for (int i = tid; i < L; i += VGPU_BLOCK) {
        const uint64_t k = ekey(i);
        if (k <= K64) {
            const uint32_t slot = atomicAdd(&cnt, 1u);
            if (slot < SEL_CAP) {
                keys[slot] = k;
                pay[slot] = (uint32_t)i;
            }
        }
    }
    __syncthreads();
    const int n2 = next_pow2(Pe);
    for (int t = Pe + tid; t < n2; t += VGPU_BLOCK) {
        keys[t] = ~0ull;
        pay[t] = 0xffffffffu;
    }
    block_bitonic_sort(keys, pay, n2);
    for (int p = tid; p < Pe; p += VGPU_BLOCK) probe[(size_t)q * P + p] = pay[p];
}

// One query per workgroup, or (flag_list != null) the queries the wave kernel
// could not finish, walked by a small grid.
template <int EPT>
__global__ __launch_bounds__(256) void coarse_select_reg_kernel(
    float* __restrict__ D, const float* __restrict__ qn, const float* __restrict__ qnorm,
    const float* __restrict__ C, int nq, int L, int d, int P, float cmax,
    uint32_t* __restrict__ probe, unsigned int* overflow, const uint32_t* flag_list,
    const uint32_t* flag_count) {
    if (!flag_list) {
        const int q = blockIdx.x;
        if (q < nq)
            select_block_query<EPT>(D + (size_t)q * L, qn + (size_t)q * d, qnorm[q], C, q, L, d, P, cmax,
                                    probe, overflow);
        return;
    }
    const uint32_t nf = *flag_count;  // written by the wave kernel before this launch
    for (uint32_t i = blockIdx.x; i < nf; i += gridDim.x) {
        __syncthreads();
        const int q = (int)flag_list[i];
        select_block_query<EPT>(D + (size_t)q * L, qn + (size_t)q * d, qnorm[q], C, q, L, d, P, cmax,
                                probe, overflow);
    }
}

// Queries whose fused-kernel candidate set may be incomplete (a lane's key
// list overflowed: many lists tie or crowd the window): approximate dot
// products of all L lists (approx_dot, within the same bound coarse_tau
// covers), then the block selection (window, exact rescoring) on them.
// With a scratch row per query (fdots, COARSE_FLAG_PAR rows of L), the first
// COARSE_FLAG_PAR flagged queries spread their dot products over the grid in
// slices of 256 lists; the workgroup that finishes a query's last slice
// (counted in fdone[fi], which it resets) runs the selection on the row.
// Flagged queries past those, or all of them without scratch, are one
// workgroup each: their dot products go to LDS.  The grid walks the flagged
// list.
template <int EPT>
__global__ __launch_bounds__(256) void coarse_exact_flagged_kernel(
    const float* __restrict__ qn, const float* __restrict__ qnorm, const float* __restrict__ C, int L,
    int d, int P, float cmax, uint32_t* __restrict__ probe, unsigned int* overflow,
    const uint32_t* flag_list, const uint32_t* flag_count, float* __restrict__ fdots, uint32_t* fdone) {
    extern __shared__ __align__(16) float qs[];  // [d rounded up to 4] query, then [L] dots
    __shared__ uint32_t last;
    float* xrow = qs + ((d + 3) & ~3);
    const uint32_t nf = *flag_count;  // written by the top-P kernel before this launch
    const uint32_t npar = fdots ? (nf < COARSE_FLAG_PAR ? nf : COARSE_FLAG_PAR) : 0u;
    const int S = (L + VGPU_BLOCK - 1) / VGPU_BLOCK;  // slices of 256 lists
    for (uint32_t it = blockIdx.x; it < npar * (uint32_t)S; it += gridDim.x) {
        __syncthreads();
        const uint32_t fi = it / (uint32_t)S;
        const int c = (int)(it % (uint32_t)S) * VGPU_BLOCK + threadIdx.x;
        const int q = (int)flag_list[fi];
        for (int j = threadIdx.x; j < d; j += VGPU_BLOCK) qs[j] = qn[(size_t)q * d + j];
        __syncthreads();
        float* row = fdots + (size_t)fi * L;
        if (c < L) row[c] = approx_dot(qs, C + (size_t)c * d, d);
        __threadfence();  // the slice is visible before it is counted
        __syncthreads();
        if (threadIdx.x == 0) {
            last = atomicAdd(&fdone[fi], 1u) == (uint32_t)(S - 1) ? 1u : 0u;
            if (last) atomicExch(&fdone[fi], 0u);  // every slice counted: ready for the next launch
        }
        __syncthreads();
        if (last) {
            __threadfence();  // the other workgroups' slices
            select_block_query<EPT>(row, qs, qnorm[q], C, q, L, d, P, cmax, probe, overflow);
        }
    }
    for (uint32_t fi = npar + blockIdx.x; fi < nf; fi += gridDim.x) {
        __syncthreads();
        const int q = (int)flag_list[fi];
        for (int j = threadIdx.x; j < d; j += VGPU_BLOCK) qs[j] = qn[(size_t)q * d + j];
        __syncthreads();
        int i0 = threadIdx.x;
        if ((d & 31) == 0) {  // four rows per thread with their loads in flight together
            for (; i0 + 3 * VGPU_BLOCK < L; i0 += 4 * VGPU_BLOCK) {
                float x[4];
                approx_dot_rows<4>(qs, C + (size_t)i0 * d, (size_t)VGPU_BLOCK * d, d, x);
#pragma unroll
                for (int r = 0; r < 4; r++) xrow[i0 + r * VGPU_BLOCK] = x[r];
            }
        }
        for (int i = i0; i < L; i += VGPU_BLOCK) xrow[i] = approx_dot(qs, C + (size_t)i * d, d);
        __syncthreads();
        select_block_query<EPT>(xrow, qs, qnorm[q], C, q, L, d, P, cmax, probe, overflow);
    }
}

void launch_coarse_exact_flagged(const float* qn, const float* qnorm, const float* C, int nq, int L,
                                 int d, int P, float cmax, uint32_t* probe, unsigned int* overflow,
                                 const uint32_t* flag_list, const uint32_t* flag_count, hipStream_t s,
                                 float* fdots, uint32_t* fdone) {
    if (nq <= 0) return;
    const size_t lds = ((size_t)L + ((d + 3) & ~3)) * sizeof(float);
    // flagged queries are rare: a small grid keeps the usual empty launch cheap
    const int gmax = fdots ? 256 : 64;
    const dim3 grid(nq < gmax ? nq : gmax);
    if (L <= 16 * VGPU_BLOCK) {
        ensure_dyn_lds((const void*)coarse_exact_flagged_kernel<16>, lds);
        hipLaunchKernelGGL(coarse_exact_flagged_kernel<16>, grid, dim3(256), lds, s, qn, qnorm, C, L, d, P,
                           cmax, probe, overflow, flag_list, flag_count, fdots, fdone);
    } else if (L <= 32 * VGPU_BLOCK) {
        ensure_dyn_lds((const void*)coarse_exact_flagged_kernel<32>, lds);
        hipLaunchKernelGGL(coarse_exact_flagged_kernel<32>, grid, dim3(256), lds, s, qn, qnorm, C, L, d, P,
                           cmax, probe, overflow, flag_list, flag_count, fdots, fdone);
    } else {
        ensure_dyn_lds((const void*)coarse_exact_flagged_kernel<64>, lds);
        hipLaunchKernelGGL(coarse_exact_flagged_kernel<64>, grid, dim3(256), lds, s, qn, qnorm, C, L, d, P,
                           cmax, probe, overflow, flag_list, flag_count, fdots, fdone);
    }
}

// One wave per query (four independent queries per workgroup, no block
// barriers), for L <= 4096 and Pe <= 64: 64 scores per lane in registers.  The
// Pe-th smallest of the 64 lane minima bounds the Pe-th smallest score (Pe
// distinct lanes hold a score at or below it), so every list whose exact score
// can be among the Pe smallest has approximate score <= that bound + 2 tau.
// The window is rescored exactly and sorted in registers.  A window of more
// than WSEL_CAP lists (degenerate inputs) sends the query to the block kernel.
#define WSEL_CAP 256
#define WSEL_QD 512

__global__ __launch_bounds__(256) void coarse_select_wave_kernel(
    const float* __restrict__ D, const float* __restrict__ qn, const float* __restrict__ qnorm,
    const float* __restrict__ C, int nq, int L, int d, int P, float cmax,
    uint32_t* __restrict__ probe, uint32_t* __restrict__ flag_list, uint32_t* flag_count) {
    __shared__ uint64_t wkeys[4][WSEL_CAP];
    __shared__ float wq[4][WSEL_QD];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int q = blockIdx.x * 4 + wave;
    if (q >= nq) return;  // per wave: no block barriers below
    const float* row = D + (size_t)q * L;
    const int Pe = P < L ? P : L;
    // element (t, j) of a lane is score 256 t + 4 lane + j; loads clamped in bounds
    uint32_t fk[64];
    uint32_t mn = 0xffffffffu;
#pragma unroll
    for (int t = 0; t < 16; t++) {
        const int b = 256 * t + 4 * lane;
        const int bc = b + 4 <= L ? b : (L >= 4 ? ((L - 4) & ~3) : 0);
        float x[4];
        if ((L & 3) == 0 && L >= 4) {
            const float4 v = *reinterpret_cast<const float4*>(row + bc);
            x[0] = v.x; x[1] = v.y; x[2] = v.z; x[3] = v.w;
        } else {
#pragma unroll
            for (int j = 0; j < 4; j++) x[j] = row[b + j < L ? b + j : L - 1];
        }
#pragma unroll
        for (int j = 0; j < 4; j++) {
            fk[4 * t + j] = b + j < L ? fkey(1.0f - x[j]) : 0xffffffffu;
            mn = fk[4 * t + j] < mn ? fk[4 * t + j] : mn;
        }
    }
    uint64_t km[1] = {mn};
    wave_sort_regs<1>(km);
    const uint32_t T = (uint32_t)__shfl(km[0], Pe - 1, 64);
    const float W = fkey_to_float(T) + 2.0f * coarse_tau(d, qnorm[q], cmax);
    uint32_t WK = fkey(W);
    WK = WK < 0xfffffffeu ? WK + 1u : 0xffffffffu;  // one ulp to spare
    if (WK < T) WK = T;
    uint32_t cnt = 0;
    uint64_t* wk = wkeys[wave];
#pragma unroll
    for (int t = 0; t < 16; t++) {
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const bool take = 256 * t + 4 * lane + j < L && fk[4 * t + j] <= WK;
            const uint64_t m = __ballot(take);
            const uint32_t below =
                __builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0u));
            if (take && cnt + below < WSEL_CAP) wk[cnt + below] = (uint64_t)(256 * t + 4 * lane + j);
            cnt += (uint32_t)__popcll(m);
        }
    }
    if (cnt > WSEL_CAP) {
        if (lane == 0) flag_list[atomicAdd(flag_count, 1u)] = (uint32_t)q;
        return;
    }
    float* qs = wq[wave];
    for (int j = lane; j < d; j += 64) qs[j] = qn[(size_t)q * d + j];
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
    __builtin_amdgcn_wave_barrier();
    uint64_t k4[4];
#pragma unroll
    for (int e = 0; e < 4; e++) {
        const uint32_t t = e * 64 + lane;
        k4[e] = ~0ull;
        if (t < cnt) {
            const uint32_t c = (uint32_t)wk[t];
            k4[e] = cand_key(1.0f - seq_dot_stream(qs, C + (size_t)c * d, d), c);
        }
    }
    if (cnt <= 64) {
        uint64_t k1[1] = {k4[0]};
        wave_sort_regs<1>(k1);
        if (lane < Pe) probe[(size_t)q * P + lane] = (uint32_t)k1[0];
    } else if (cnt <= 128) {
        uint64_t k2[2] = {k4[0], k4[1]};
        wave_sort_regs<2>(k2);
#pragma unroll
        for (int e = 0; e < 2; e++)
            if (e * 64 + lane < Pe) probe[(size_t)q * P + e * 64 + lane] = (uint32_t)k2[e];
    } else {
        wave_sort_regs<4>(k4);
#pragma unroll
        for (int e = 0; e < 4; e++)
            if (e * 64 + lane < Pe) probe[(size_t)q * P + e * 64 + lane] = (uint32_t)k4[e];
    }
}

// Generic selection (any L): radix select over the score row in global memory.
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

// Selection of more than SEL_CAP lists (P up to L <= SEL_WIDE_MAX): the exact
// score of every list (the reference's sequential 1 - dot,
// cosine_distance_normalized) into the row, an exact 64-bit radix select of
// the Pe-th (score, list) key, then the Pe keys at or below it sorted in LDS
// (search.rs:1602-1617 with nprobe up to num_clusters).
__global__ __launch_bounds__(256) void coarse_select_wide_kernel(float* __restrict__ D,
                                                                 const float* __restrict__ qn,
                                                                 const float* __restrict__ C, int nq,
                                                                 int L, int d, int P,
                                                                 uint32_t* __restrict__ probe) {
    extern __shared__ __align__(16) uint64_t wide_keys[];  // [next_pow2(Pe)]
    __shared__ RadixScratch rs;
    __shared__ uint32_t cnt;
    const int tid = threadIdx.x;
    const int q = blockIdx.x;
    if (q >= nq) return;
    float* row = D + (size_t)q * L;
    const float* qv = qn + (size_t)q * d;
    const int Pe = P < L ? P : L;
    for (int i = tid; i < L; i += blockDim.x) row[i] = 1.0f - seq_dot(qv, C + (size_t)i * d, d);
    __threadfence_block();
    __syncthreads();
    auto ekey = [&](int i) -> uint64_t { return cand_key(row[i], (uint32_t)i); };
    const uint64_t K64 = Pe < L ? block_radix_select<uint64_t>(ekey, L, (uint32_t)(Pe - 1), &rs) : ~0ull;
    if (tid == 0) cnt = 0;
    __syncthreads();
    for (int i = tid; i < L; i += blockDim.x) {
        const uint64_t k = ekey(i);
        if (k <= K64) {
            const uint32_t slot = atomicAdd(&cnt, 1u);
            if (slot < (uint32_t)Pe) wide_keys[slot] = k;
        }
    }
    __syncthreads();
    const int n2 = next_pow2(Pe);
    for (int t = Pe + tid; t < n2; t += blockDim.x) wide_keys[t] = ~0ull;
    block_bitonic_sort_keys(wide_keys, n2);
    for (int p = tid; p < Pe; p += blockDim.x) probe[(size_t)q * P + p] = (uint32_t)wide_keys[p];
}

void launch_coarse_select_wide(float* D, const float* qn, const float* C, int nq, int L, int d, int P,
                               uint32_t* probe, hipStream_t s) {
    if (nq <= 0) return;
    const int Pe = P < L ? P : L;
    size_t n2 = 1;
    while (n2 < (size_t)Pe) n2 <<= 1;
    const size_t lds = n2 * sizeof(uint64_t);
    ensure_dyn_lds((const void*)coarse_select_wide_kernel, lds);
    hipLaunchKernelGGL(coarse_select_wide_kernel, dim3(nq), dim3(256), lds, s, D, qn, C, nq, L, d, P, probe);
}

void launch_coarse_select(float* D, const float* qn, const float* qnorm, const float* C, int nq,
                          int L, int d, int P, float cmax, uint32_t* probe,
                          unsigned int* overflow, uint32_t* flag_list, uint32_t* flag_count,
                          hipStream_t s) {
    if (nq <= 0) return;
    const int Pe = P < L ? P : L;
    if (d > SEL_CAP || Pe > 256 || L > 64 * VGPU_BLOCK) {
        hipLaunchKernelGGL(coarse_select_kernel, dim3(nq), dim3(256), 0, s, D, qn, qnorm, C, nq, L, d,
                           P, cmax, probe, overflow);
        return;
    }
    auto block = L <= 16 * VGPU_BLOCK   ? coarse_select_reg_kernel<16>
                 : L <= 32 * VGPU_BLOCK ? coarse_select_reg_kernel<32>
                                        : coarse_select_reg_kernel<64>;
    if (L <= 4096 && Pe <= 64 && d <= WSEL_QD) {
        hipLaunchKernelGGL(coarse_select_wave_kernel, dim3((nq + 3) / 4), dim3(256), 0, s, D, qn, qnorm,
                           C, nq, L, d, P, cmax, probe, flag_list, flag_count);
        hipLaunchKernelGGL(block, dim3(nq < 128 ? nq : 128), dim3(256), 0, s, D, qn, qnorm, C, nq, L,
                           d, P, cmax, probe, overflow, flag_list, flag_count);
        return;
    }
    hipLaunchKernelGGL(block, dim3(nq), dim3(256), 0, s, D, qn, qnorm, C, nq, L, d, P, cmax, probe,
                       overflow, nullptr, nullptr);
}

}  // namespace vgpu
