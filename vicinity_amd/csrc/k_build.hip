// Build-side kernels: residual PQ encode, the per-entry FAST term b(x), the
// FastScan nibble packing, and the per-kernel LUT test entry.
//
// Reference: quantize src/ivf_pq/pq.rs:136-161 (argmin over codewords of the
// squared L2 distance, strict `<`, lowest code wins); residuals v - c
// src/ivf_pq/search.rs:722-729; PackedCodes4bit::pack src/pq_simd.rs:426-486;
// compute_adc_table_into pq.rs:196-266.
#include "vgpu_device.h"
#include "vgpu_launch.h"

namespace vgpu {

// codes[i*M + m] for one subspace per grid row.  r_j = x_j - c_j (or x_j when
// there is no centroid), dist = sum_j (r_j - cw_j)^2 in order.
template <int DS>
__global__ __launch_bounds__(256) void encode_kernel(const float* __restrict__ x, int n, int d,
                                                     const float* __restrict__ centroids,
                                                     const uint32_t* __restrict__ assign,
                                                     const float* __restrict__ cb, int M, int K,
                                                     int ds, uint8_t* __restrict__ codes) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    const int m = blockIdx.y;
    if (i >= n) return;
    const float* xs = x + (size_t)i * d + m * ds;
    const float* cs = centroids ? centroids + (size_t)assign[i] * d + m * ds : nullptr;
    const float* cbm = cb + (size_t)m * K * ds;
    int best = 0;
    float best_d = __int_as_float(0x7f800000);
    if constexpr (DS > 0) {
        float r[DS];
#pragma unroll
        for (int j = 0; j < DS; j++) r[j] = cs ? xs[j] - cs[j] : xs[j];
        for (int k = 0; k < K; k++) {
            const float* cw = cbm + (size_t)k * DS;
            float s = 0.0f;
#pragma unroll
            for (int j = 0; j < DS; j++) {
                float t = r[j] - cw[j];
                s += t * t;
            }
            if (s < best_d) {
                best_d = s;
                best = k;
            }
        }
    } else {
        for (int k = 0; k < K; k++) {
            const float* cw = cbm + (size_t)k * ds;
            float s = 0.0f;
            for (int j = 0; j < ds; j++) {
                float rj = cs ? xs[j] - cs[j] : xs[j];
                float t = rj - cw[j];
                s += t * t;
            }
            if (s < best_d) {
                best_d = s;
                best = k;
            }
        }
    }
    codes[(size_t)i * M + m] = (uint8_t)(best < 255 ? best : 255);
}

void launch_encode(const float* x, int n, int d, const float* centroids, const uint32_t* assign,
                   const float* codebooks, int M, int K, int ds, uint8_t* codes, hipStream_t s) {
    if (n <= 0) return;
    dim3 grid((n + 255) / 256, M);
#define ENC(DSV) hipLaunchKernelGGL(encode_kernel<DSV>, grid, dim3(256), 0, s, x, n, d, centroids, \
                                    assign, codebooks, M, K, ds, codes)
    switch (ds) {
        case 1: ENC(1); break;
        case 2: ENC(2); break;
        case 4: ENC(4); break;
        case 8: ENC(8); break;
        case 16: ENC(16); break;
        default: ENC(0); break;
    }
#undef ENC
}

// b(x) = sum_m (||cw||^2 + 2 c_m . cw) for the entry at each list position.
__global__ void bias_kernel(DevIndex ix, float* __restrict__ bias) {
    const uint32_t pos = blockIdx.x * blockDim.x + threadIdx.x;
    if (pos >= ix.n) return;
    int lo = 0, hi = ix.L;  // find l with off[l] <= pos < off[l+1]
    while (hi - lo > 1) {
        int mid = (lo + hi) >> 1;
        if (ix.offsets[mid] <= pos) lo = mid;
        else hi = mid;
    }
    const float* c = ix.centroids + (size_t)lo * ix.d;
    const uint8_t* row = ix.codes + (size_t)pos * ix.M;
    float b = 0.0f;
    for (int m = 0; m < ix.M; m++) {
        const float* cw = ix.codebooks + ((size_t)m * ix.K + row[m]) * ix.ds;
        float e1 = 0.0f, e2 = 0.0f;
        for (int j = 0; j < ix.ds; j++) {
            e1 += cw[j] * cw[j];
            e2 += c[m * ix.ds + j] * cw[j];
        }
        b += e1 + 2.0f * e2;
    }
    bias[pos] = b;
}

void launch_bias(const DevIndex& ix, float* bias, hipStream_t s) {
    if (ix.n == 0) return;
    hipLaunchKernelGGL(bias_kernel, dim3((ix.n + 255) / 256), dim3(256), 0, s, ix, bias);
}

// One workgroup per list, one thread per 4-byte word of the list's blocks.
__global__ void tblocks_kernel(DevIndex ix, uint8_t* __restrict__ out) {
    const int l = blockIdx.x;
    const uint32_t beg = ix.offsets[l], len = ix.offsets[l + 1] - beg;
    const uint32_t b0 = ix.tblk_off[l], nb = ix.tblk_off[l + 1] - b0;
    const uint32_t M = (uint32_t)ix.M, blk = (uint32_t)TBLK_BYTES(M), cb = 16u * M;
    uint32_t* o = reinterpret_cast<uint32_t*>(out + (size_t)b0 * blk);
    for (uint32_t w = threadIdx.x; w < nb * blk / 4u; w += blockDim.x) {
        const uint32_t b = w / (blk / 4u), within = (w % (blk / 4u)) * 4u;
        uint32_t word = 0u;
        if (within < cb) {
            const uint32_t m = within / 16u;
            for (uint32_t i = 0; i < 4u; i++) {
                const uint32_t j = within % 16u + i, e = b * 16u + (j ^ (m & 15u));
                const uint32_t c = e < len ? ix.codes[(size_t)(beg + e) * M + m] : 0u;
                word |= c << (8u * i);
            }
        } else {
            const uint32_t e = b * 16u + (within - cb) / 4u;
            word = e < len ? __float_as_uint(ix.bias[beg + e]) : 0u;
        }
        o[w] = word;
    }
}

void launch_tblocks(const DevIndex& ix, uint8_t* tblocks, hipStream_t s) {
    if (ix.L <= 0) return;
    hipLaunchKernelGGL(tblocks_kernel, dim3(ix.L), dim3(256), 0, s, ix, tblocks);
}

// One workgroup per list; lists shorter than 16 entries have no blocks
// (they take the exact float path, search.rs:1355-1375).
__global__ void pack4_kernel(DevIndex ix, uint8_t* __restrict__ packed) {
    const int l = blockIdx.x;
    const uint32_t beg = ix.offsets[l], len = ix.offsets[l + 1] - beg;
    const uint32_t nb = ix.pack_off[l + 1] - ix.pack_off[l];
    if (nb == 0) return;
    const int M = ix.M;
    uint8_t* out = packed + (size_t)ix.pack_off[l] * 16 * M;
    const uint32_t total = nb * 16u * M;
    for (uint32_t e = threadIdx.x; e < total; e += blockDim.x) {
        uint32_t b = e / (16u * M), rem = e % (16u * M);
        uint32_t m = rem / 16u, lane = rem % 16u;
        uint32_t lo = b * 32u + lane, hi = lo + 16u;
        uint8_t clo = lo < len ? (ix.codes[(size_t)(beg + lo) * M + m] & 0x0F) : 0;
        uint8_t chi = hi < len ? (ix.codes[(size_t)(beg + hi) * M + m] & 0x0F) : 0;
        out[e] = (uint8_t)(clo | (chi << 4));
    }
}

void launch_pack4(const DevIndex& ix, uint8_t* packed, hipStream_t s) {
    if (ix.L <= 0) return;
    hipLaunchKernelGGL(pack4_kernel, dim3(ix.L), dim3(256), 0, s, ix, packed);
}

// tables[t*M*K + m*K + k] = sum_j (r_tj - cw_j)^2 (pq.rs:232-251 order).
__global__ void adc_tables_kernel(const float* __restrict__ cb, int M, int K, int ds,
                                  const float* __restrict__ r, int nr, float* __restrict__ tables) {
    const size_t e = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    const size_t per = (size_t)M * K;
    if (e >= per * nr) return;
    const size_t t = e / per, mk = e % per;
    const int m = (int)(mk / K);
    const float* rr = r + t * (size_t)M * ds + (size_t)m * ds;
    const float* cw = cb + mk * ds;
    float acc = 0.0f;
    for (int j = 0; j < ds; j++) {
        float diff = rr[j] - cw[j];
        acc += diff * diff;
    }
    tables[e] = acc;
}

void launch_adc_tables(const float* codebooks, int M, int K, int ds, const float* r, int nr,
                       float* tables, hipStream_t s) {
    size_t total = (size_t)M * K * nr;
    if (total == 0) return;
    hipLaunchKernelGGL(adc_tables_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, s,
                       codebooks, M, K, ds, r, nr, tables);
}

// Lloyd update of every active key (k-means centroid, or codeword c of
// subspace m): the float64 sum of its members' rows in index order, the mean
// cast to float, and with NORM the row normalised like normalize_row (float
// sum of squares in order, sqrt, divide when the norm exceeds 1e-10).  An empty
// key keeps its row.  One wave per key: lanes test 64 rows per step, a ballot
// lists the members, and each member's row is added in row order, lane j owning
// dims j, j + 64, ...  Labels: u32 per row (U8 false) or the code byte of
// subspace m at labels[i * M + m] (U8 true).  Rows: x[i * d + col0], w floats
// wide (w <= 256); out rows are w floats at out[key * w].
template <bool U8, bool NORM>
__global__ __launch_bounds__(256) void kmeans_update_kernel(const float* __restrict__ x, int n, int d,
                                                            int w, int M, const void* __restrict__ labels,
                                                            int K, const uint8_t* __restrict__ active,
                                                            float* __restrict__ out) {
    const int lane = threadIdx.x & 63;
    const int key = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (key >= M * K) return;
    const int m = key / K, c = key - m * K;
    if (active && !active[m]) return;
    const size_t col0 = U8 ? (size_t)m * w : 0;
    double acc[4] = {0.0, 0.0, 0.0, 0.0};
    uint32_t count = 0;
    for (int i0 = 0; i0 < n; i0 += 64) {
        const int i = i0 + lane;
        bool mine = false;
        if (i < n) {
            mine = U8 ? ((const uint8_t*)labels)[(size_t)i * M + m] == (uint8_t)c
                      : ((const uint32_t*)labels)[i] == (uint32_t)c;
        }
        uint64_t b = __ballot(mine);
        count += (uint32_t)__popcll(b);
        while (b) {
            const int src = __ffsll((unsigned long long)b) - 1;
            b &= b - 1;
            const float* xr = x + (size_t)(i0 + src) * d + col0;
#pragma unroll
            for (int t = 0; t < 4; t++) {
                const int j = lane + 64 * t;
                if (j < w) acc[t] += (double)xr[j];
            }
        }
    }
    if (count == 0) return;
    float f[4];
#pragma unroll
    for (int t = 0; t < 4; t++) f[t] = (float)(acc[t] / (double)count);
    if constexpr (NORM) {
        float s2 = 0.0f;
        for (int j = 0; j < w; j++) {  // uniform loop: every lane forms the same sum
            const float v = __shfl(f[j >> 6], j & 63, 64);
            s2 += v * v;
        }
        const float nrm = sqrtf(s2);
        if (nrm > 1e-10f) {
#pragma unroll
            for (int t = 0; t < 4; t++) f[t] = f[t] / nrm;
        }
    }
    float* o = out + (size_t)key * w;
#pragma unroll
    for (int t = 0; t < 4; t++) {
        const int j = lane + 64 * t;
        if (j < w) o[j] = f[t];
    }
}

void launch_kmeans_update(const float* x, int n, int d, int w, int M, const void* labels, bool u8,
                          int K, const uint8_t* active, bool normalize, float* out, hipStream_t s) {
    const dim3 grid((unsigned)(((size_t)M * K + 3) / 4));
    if (u8)
        hipLaunchKernelGGL((kmeans_update_kernel<true, false>), grid, dim3(256), 0, s, x, n, d, w, M,
                           labels, K, active, out);
    else if (normalize)
        hipLaunchKernelGGL((kmeans_update_kernel<false, true>), grid, dim3(256), 0, s, x, n, d, w, M,
                           labels, K, active, out);
    else
        hipLaunchKernelGGL((kmeans_update_kernel<false, false>), grid, dim3(256), 0, s, x, n, d, w, M,
                           labels, K, active, out);
}

}  // namespace vgpu
