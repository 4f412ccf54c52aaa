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

// One workgroup per list, one thread per 4-byte word of the list's lane
// records: M bytes of codes per record (codebooks m, m + 16, ...: byte j is
// the code of entry j ^ m), then one b(x) per record.
__global__ void tblocks_kernel(DevIndex ix, uint8_t* __restrict__ tcodes, float* __restrict__ tbias) {
    const int l = blockIdx.x;
    const uint32_t beg = ix.offsets[l], len = ix.offsets[l + 1] - beg;
    const uint32_t b0 = ix.tblk_off[l], nb = ix.tblk_off[l + 1] - b0;
    const uint32_t M = (uint32_t)ix.M;
    uint32_t* o = reinterpret_cast<uint32_t*>(tcodes + (size_t)b0 * 16u * M);
    for (uint32_t w = threadIdx.x; w < nb * 4u * M; w += blockDim.x) {
        const uint32_t rec = w / (M / 4u), r = (w % (M / 4u)) * 4u;  // lane record, byte within
        const uint32_t b = rec / 16u, mm = rec % 16u;
        const uint32_t m = (r / 16u) * 16u + mm;  // codebook
        uint32_t word = 0u;
        for (uint32_t i = 0; i < 4u; i++) {
            const uint32_t j = r % 16u + i, e = b * 16u + (j ^ mm);
            const uint32_t c = e < len ? ix.codes[(size_t)(beg + e) * M + m] : 0u;
            word |= c << (8u * i);
        }
        o[w] = word;
    }
    // padding entries get a NaN b(x): their approximate distance is NaN,
    // which no filter takes
    for (uint32_t e = threadIdx.x; e < nb * 16u; e += blockDim.x)
        tbias[(size_t)b0 * 16u + e] = e < len ? ix.bias[beg + e] : __int_as_float(0x7fc00000);
}

void launch_tblocks(const DevIndex& ix, uint8_t* tcodes, float* tbias, hipStream_t s) {
    if (ix.L <= 0) return;
    hipLaunchKernelGGL(tblocks_kernel, dim3(ix.L), dim3(256), 0, s, ix, tcodes, tbias);
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

// ---- Lloyd update over per-key member lists.
//
// Every active key (k-means centroid, or codeword c of subspace m; global key
// m * K + c) becomes the float64 sum of its members' rows in row order, the
// mean cast to float, and with NORM the row normalised like normalize_row
// (float sum of squares in order, sqrt, divide when the norm exceeds 1e-10).
// An empty key keeps its row.  Labels: u32 per row (M = 1) or the code byte of
// subspace m at labels[i * M + m]; rows x[i * d + m * w .. + w), w <= 256;
// out rows are w floats at out[key * w].
//
// The member lists come from a stable counting sort of the labels, built
// once per update instead of one scan of every label per key:
//   count   rows in blocks of R; cnt[key * nb + b] = members of key in block b
//           (non-returning atomics);
//   bscan   one wave per key: cnt row -> exclusive prefix over blocks, the
//           key's total to tot[key];
//   tscan   one workgroup: tot -> exclusive prefix over keys, tot[keys] = sum;
//   scatter one workgroup per (block, subspace): the block's (label, row)
//           pairs sorted in LDS; a pair at sorted position p lands at
//           tot[key] + cnt[key * nb + b] + (p - first position of its label),
//           so each key's list holds its rows in ascending order;
//   update  one wave per key walks its list in order.
#define KM_THREADS 256

struct KmSort {
    int R, nb;            // rows per block (power of two, 1024..4096), blocks
    size_t keys;          // M * K
    uint32_t* cnt;        // [keys * nb]
    uint32_t* tot;        // [keys + 1]
    uint32_t* members;    // [M * n]
};

static KmSort km_layout(int n, int M, int K, uint32_t* base) {
    KmSort k;
    k.keys = (size_t)M * K;
    k.R = 1024;
    // larger blocks when the count table would pass 2^25 words
    while (k.R < 4096 && k.keys * (((size_t)n + k.R - 1) / k.R) > ((size_t)1 << 25)) k.R <<= 1;
    k.nb = (int)(((size_t)n + k.R - 1) / k.R);
    k.cnt = base;
    k.tot = k.cnt + k.keys * k.nb;
    k.members = k.tot + k.keys + 1;
    return k;
}

size_t kmeans_update_scratch_words(int n, int M, int K) {
    const KmSort k = km_layout(n, M, K, nullptr);
    return k.keys * k.nb + k.keys + 1 + (size_t)M * n + 1;  // + 1: even length for the clear
}

template <bool U8>
__device__ __forceinline__ uint32_t km_label(const void* labels, int i, int M, int m) {
    return U8 ? (uint32_t)((const uint8_t*)labels)[(size_t)i * M + m] : ((const uint32_t*)labels)[i];
}

template <bool U8>
__global__ __launch_bounds__(KM_THREADS) void km_count_kernel(const void* __restrict__ labels, int n, int M,
                                                              int K, const uint8_t* __restrict__ active,
                                                              int R, int nb, uint32_t* __restrict__ cnt) {
    const int b = blockIdx.x, m = blockIdx.y;
    if (active && !active[m]) return;
    const int i1 = min(n, (b + 1) * R);
    for (int i = b * R + threadIdx.x; i < i1; i += KM_THREADS) {
        const uint32_t c = km_label<U8>(labels, i, M, m);
        atomicAdd(&cnt[((size_t)m * K + c) * nb + b], 1u);
    }
}

__global__ __launch_bounds__(KM_THREADS) void km_bscan_kernel(uint32_t* __restrict__ cnt, int nb, size_t keys,
                                                              uint32_t* __restrict__ tot) {
    const int lane = threadIdx.x & 63;
    const size_t key = (size_t)blockIdx.x * (KM_THREADS / 64) + (threadIdx.x >> 6);
    if (key >= keys) return;
    uint32_t* row = cnt + key * nb;
    uint32_t carry = 0;
    for (int b0 = 0; b0 < nb; b0 += 64) {
        const int b = b0 + lane;
        const uint32_t v = b < nb ? row[b] : 0u;
        uint32_t incl = v;
#pragma unroll
        for (int o = 1; o < 64; o <<= 1) {
            const uint32_t t = __shfl_up(incl, o, 64);
            if (lane >= o) incl += t;
        }
        if (b < nb) row[b] = carry + incl - v;
        carry += __shfl(incl, 63, 64);
    }
    if (lane == 0) tot[key] = carry;
}

// One workgroup of 1024 threads: tot[0 .. keys) -> exclusive prefix, tot[keys] = total.
__global__ __launch_bounds__(1024) void km_tscan_kernel(uint32_t* __restrict__ tot, size_t keys) {
    __shared__ uint32_t wsum[16];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    uint32_t carry = 0;
    for (size_t i0 = 0; i0 < keys; i0 += 1024) {
        const size_t i = i0 + tid;
        const uint32_t v = i < keys ? tot[i] : 0u;
        uint32_t incl = v;
#pragma unroll
        for (int o = 1; o < 64; o <<= 1) {
            const uint32_t t = __shfl_up(incl, o, 64);
            if (lane >= o) incl += t;
        }
        if (lane == 63) wsum[wave] = incl;
        __syncthreads();
        uint32_t before = carry, all = 0;
#pragma unroll
        for (int w = 0; w < 16; w++) {
            const uint32_t s = wsum[w];
            before += w < wave ? s : 0u;
            all += s;
        }
        if (i < keys) tot[i] = before + incl - v;
        carry += all;
        __syncthreads();  // wsum is rewritten by the next tile
    }
    if (tid == 0) tot[keys] = carry;
}

template <bool U8>
__global__ __launch_bounds__(KM_THREADS) void km_scatter_kernel(const void* __restrict__ labels, int n, int M,
                                                                int K, const uint8_t* __restrict__ active,
                                                                int R, int nb, const uint32_t* __restrict__ cnt,
                                                                const uint32_t* __restrict__ tot,
                                                                uint32_t* __restrict__ members) {
    extern __shared__ __align__(16) uint64_t sk[];  // [R] (label << 32 | row within the block)
    const int b = blockIdx.x, m = blockIdx.y, tid = threadIdx.x;
    if (active && !active[m]) return;
    const int i0 = b * R;
    for (int t = tid; t < R; t += KM_THREADS) {
        const int i = i0 + t;
        sk[t] = i < n ? ((uint64_t)km_label<U8>(labels, i, M, m) << 32) | (uint32_t)t : ~0ull;
    }
    for (int size = 2; size <= R; size <<= 1) {
        for (int stride = size >> 1; stride > 0; stride >>= 1) {
            __syncthreads();
            for (int t = tid; t < (R >> 1); t += KM_THREADS) {
                const int a = 2 * t - (t & (stride - 1)), c = a + stride;
                const bool asc = (a & size) == 0;
                const uint64_t x = sk[a], y = sk[c];
                if ((x > y) == asc) {
                    sk[a] = y;
                    sk[c] = x;
                }
            }
        }
    }
    __syncthreads();
    for (int p = tid; p < R; p += KM_THREADS) {
        const uint64_t e = sk[p];
        if (e == ~0ull) continue;
        const uint32_t lab = (uint32_t)(e >> 32);
        // first position of this label: lower bound of (lab << 32) in sk[0 .. p]
        const uint64_t lo_key = (uint64_t)lab << 32;
        int lo = 0, hi = p;
        while (lo < hi) {
            const int mid = (lo + hi) >> 1;
            if (sk[mid] < lo_key) lo = mid + 1;
            else hi = mid;
        }
        const size_t key = (size_t)m * K + lab;
        members[tot[key] + cnt[key * nb + b] + (uint32_t)(p - lo)] = (uint32_t)(i0 + (uint32_t)e);
    }
}

// One wave per key: lane j owns dims j, j + 64, ...; members in list order.
template <bool NORM>
__global__ __launch_bounds__(KM_THREADS) void kmeans_update_kernel(const float* __restrict__ x, int d, int w,
                                                                   int M, int K,
                                                                   const uint8_t* __restrict__ active,
                                                                   const uint32_t* __restrict__ tot,
                                                                   const uint32_t* __restrict__ members,
                                                                   float* __restrict__ out) {
    const int lane = threadIdx.x & 63;
    const int key = blockIdx.x * (KM_THREADS / 64) + (threadIdx.x >> 6);
    if (key >= M * K) return;
    const int m = key / K;
    if (active && !active[m]) return;
    const uint32_t start = tot[key], count = tot[key + 1] - start;
    if (count == 0) return;
    const float* xm = x + (size_t)m * w;
    double acc[4] = {0.0, 0.0, 0.0, 0.0};
    for (uint32_t s0 = 0; s0 < count; s0 += 64) {
        const uint32_t mine = s0 + lane < count ? members[start + s0 + lane] : 0u;
        const int nn = (int)min(64u, count - s0);
        int j = 0;
        for (; j + 4 <= nn; j += 4) {  // four rows' loads in flight, added in order
            float v[4][4];
#pragma unroll
            for (int u = 0; u < 4; u++) {
                const float* xr = xm + (size_t)__shfl(mine, j + u, 64) * d;
#pragma unroll
                for (int t = 0; t < 4; t++) v[u][t] = lane + 64 * t < w ? xr[lane + 64 * t] : 0.0f;
            }
#pragma unroll
            for (int u = 0; u < 4; u++)
#pragma unroll
                for (int t = 0; t < 4; t++)
                    if (lane + 64 * t < w) acc[t] += (double)v[u][t];
        }
        for (; j < nn; j++) {
            const float* xr = xm + (size_t)__shfl(mine, j, 64) * d;
#pragma unroll
            for (int t = 0; t < 4; t++)
                if (lane + 64 * t < w) acc[t] += (double)xr[lane + 64 * t];
        }
    }
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

hipError_t launch_kmeans_update(const float* x, int n, int d, int w, int M, const void* labels, bool u8,
                                int K, const uint8_t* active, bool normalize, float* out, uint32_t* scratch,
                                size_t scratch_words, hipStream_t s) {
    if (n <= 0 || M <= 0 || K <= 0) return hipSuccess;
    if ((uint64_t)M * (uint64_t)n >= ((uint64_t)1 << 32)) return hipErrorInvalidValue;  // 32-bit member lists
    if (scratch_words < kmeans_update_scratch_words(n, M, K)) return hipErrorInvalidValue;
    const KmSort ks = km_layout(n, M, K, scratch);
    launch_zero_words(reinterpret_cast<unsigned long long*>(ks.cnt), (ks.keys * ks.nb + 1) / 2, s);
    const dim3 bm((unsigned)ks.nb, (unsigned)M);
    const size_t lds = (size_t)ks.R * sizeof(uint64_t);
    if (u8) {
        hipLaunchKernelGGL(km_count_kernel<true>, bm, dim3(KM_THREADS), 0, s, labels, n, M, K, active, ks.R,
                           ks.nb, ks.cnt);
    } else {
        hipLaunchKernelGGL(km_count_kernel<false>, bm, dim3(KM_THREADS), 0, s, labels, n, M, K, active, ks.R,
                           ks.nb, ks.cnt);
    }
    const dim3 kw((unsigned)((ks.keys + KM_THREADS / 64 - 1) / (KM_THREADS / 64)));
    hipLaunchKernelGGL(km_bscan_kernel, kw, dim3(KM_THREADS), 0, s, ks.cnt, ks.nb, ks.keys, ks.tot);
    hipLaunchKernelGGL(km_tscan_kernel, dim3(1), dim3(1024), 0, s, ks.tot, ks.keys);
    if (u8) {
        ensure_dyn_lds((const void*)km_scatter_kernel<true>, lds);
        hipLaunchKernelGGL(km_scatter_kernel<true>, bm, dim3(KM_THREADS), lds, s, labels, n, M, K, active, ks.R,
                           ks.nb, ks.cnt, ks.tot, ks.members);
    } else {
        ensure_dyn_lds((const void*)km_scatter_kernel<false>, lds);
        hipLaunchKernelGGL(km_scatter_kernel<false>, bm, dim3(KM_THREADS), lds, s, labels, n, M, K, active, ks.R,
                           ks.nb, ks.cnt, ks.tot, ks.members);
    }
    if (normalize)
        hipLaunchKernelGGL(kmeans_update_kernel<true>, kw, dim3(KM_THREADS), 0, s, x, d, w, M, K, active, ks.tot,
                           ks.members, out);
    else
        hipLaunchKernelGGL(kmeans_update_kernel<false>, kw, dim3(KM_THREADS), 0, s, x, d, w, M, K, active, ks.tot,
                           ks.members, out);
    return hipGetLastError();
}
}  // namespace vgpu
