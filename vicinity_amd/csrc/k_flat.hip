// Flat exact top-k: MFMA fp32 GEMM ranking with a fused per-query candidate
// filter, then exact rescoring of the kept candidates with the reference's
// sequential arithmetic.
//
// Reference: l2_distance_squared src/distance.rs:78-83 (scalar backend
// src/simd.rs:118-121: sum (x - y)^2 in order) and cosine_distance_normalized
// src/distance.rs:104-109 (1 - dot); brute-force ground truth
// src/ivf_pq/search.rs:3376-3392.
//
// Ranking distance (metric 0): ||x||^2 - 2 q.x (||q||^2 is constant per query);
// metric 1: 1 - q.x.  A ranking kernel keeps, for every (query, database
// slice), the kk smallest ranking keys; the merge kernel gathers the slices,
// checks that the kept set provably contains the exact top-k (gap > 2 tau)
// and rescores it; a query that fails the check is searched exhaustively with
// the exact arithmetic.
//
// flat_rank_kernel (d <= 128): bf16x3 MFMA products (q.x ~ qh.xh + qh.xl +
// ql.xh, as the coarse quantiser), 128 queries per workgroup held in
// registers, the slice's vectors streamed through LDS two 16-vector tiles at
// a time (pre-split into bf16 hi/lo, tile-major).  Each score is compared
// with its row's threshold in registers; the rare ones below it are appended
// to the row's LDS buffer, which the row's 16 lanes cut back to the kk
// smallest by a bitonic sort when it fills.  flat_partial_kernel (any d) is
// the fp32 MFMA path with per-row LDS thresholds.
#include "vgpu_device.h"
#include "vgpu_bounds.h"
#include "vgpu_launch.h"

namespace vgpu {

typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

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


// ---- bf16x3 ranking kernel (d <= 128) ------------------------------------

#define FR_TPS 2    // database tiles (16 vectors each) per pipeline stage
#define FR_QBW 2    // query blocks (16 queries each) per wave
#define FR_ROWS (4 * FR_QBW * 16)  // queries per workgroup
#define FR_J 4      // keys each lane keeps per row (and sorts per lane at the end)
#define FR_BIG 3.0e38f

// Round to nearest even bfloat16 bits (finite inputs); x = hi + lo + r with
// |r| <= 2^-16 |x|.
__device__ __forceinline__ uint32_t fr_bf16_bits(float x) {
    const uint32_t u = __float_as_uint(x);
    return (u + 0x7fffu + ((u >> 16) & 1u)) >> 16;
}

// Ascending list of the FR_J smallest keys: t_i' = med3(t_{i-1}, t_i, v) from
// the bottom, t_0' = min(t_0, v).
__device__ __forceinline__ void fr_insert(float (&t)[FR_J], float v) {
#pragma unroll
    for (int i = FR_J - 1; i > 0; i--) t[i] = __builtin_amdgcn_fmed3f(t[i - 1], t[i], v);
    t[0] = fminf(t[0], v);
}

// Workgroup (4 waves) = FR_ROWS queries x one database slice of tiles
// [blockIdx.y * tps, ..) (tps <= 2^ib).  Wave w holds query blocks
// FR_QBW w .. + FR_QBW - 1 (bf16 hi/lo A operands in registers); every stage
// of FR_TPS tiles is copied to LDS once and multiplied by all of them.  The
// lane of group g (lanes 16 g .. + 15) and column c scores rows 4 g .. + 3 of
// each of its query blocks against vector 16 tile + c and keeps, per row, the
// FR_J smallest keys (score with the low ib mantissa bits replaced by the
// tile's index in the slice).  At the end each row's 16 lanes write their
// 16 FR_J keys as (fkey, vector index), unsorted (the merge selects), and a
// bound every key the slice dropped is at or above: the FR_J-th key of every
// full lane list.
template <int DT>
__global__ __launch_bounds__(256) void flat_rank_kernel(
    const float* __restrict__ Q, int nq, int d, const uint4* __restrict__ Xb_in,
    const float* __restrict__ Xnorm, int n, int metric, int kk, int tps, int ib, int splits,
    uint64_t* __restrict__ partial, uint32_t* __restrict__ pbound) {
    extern __shared__ __align__(16) char smem[];
    constexpr int TC = 2 * DT * 64;  // 16-byte chunks per tile (hi, then lo)
    constexpr int SC = FR_TPS * TC;  // chunks per stage
    constexpr int PER = SC / VGPU_BLOCK;
    static_assert(SC % VGPU_BLOCK == 0, "stage split");
    u32x4* stage = reinterpret_cast<u32x4*>(smem);                // [2][SC]
    float* snorm = reinterpret_cast<float*>(smem + 2 * SC * 16);  // [2][FR_TPS * 16]
    const u32x4* Xb = reinterpret_cast<const u32x4*>(Xb_in);
    const int tid = threadIdx.x, lane = tid & 63, g = lane >> 4, c = lane & 15;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int q0 = blockIdx.x * FR_ROWS, sl = blockIdx.y;
    const int ntiles = (n + 15) / 16;
    const int tile0 = sl * tps, tile1 = min(ntiles, tile0 + tps);
    const int nst = tile1 > tile0 ? (tile1 - tile0 + FR_TPS - 1) / FR_TPS : 0;
    const uint32_t kmask = ~((1u << ib) - 1u);

    // A operands: row (FR_QBW wave + qb) * 16 + c of the block, dimensions
    // 32 t + 8 g .. + 7 (zero past d; rows past nq repeat the last query and
    // are never written).
    u32x4 ah[FR_QBW][DT], al[FR_QBW][DT];
    const float qsc = metric == 0 ? -2.0f : -1.0f;
#pragma unroll
    for (int qb = 0; qb < FR_QBW; qb++) {
        const int row = min(q0 + (FR_QBW * wave + qb) * 16 + c, nq - 1);
        const float* qr = Q + (size_t)row * d;
#pragma unroll
        for (int t = 0; t < DT; t++) {
            uint32_t hb[8], lb[8];
#pragma unroll
            for (int i = 0; i < 8; i++) {
                const int j = 32 * t + 8 * g + i;
                // scaled by -2 (metric 0) or -1 (exact), so an accumulator is
                // the score less ||x||^2 (or less 1)
                const float x = j < d ? qsc * qr[j] : 0.0f;
                hb[i] = fr_bf16_bits(x);
                lb[i] = fr_bf16_bits(x - __uint_as_float(hb[i] << 16));
            }
            ah[qb][t] = u32x4{hb[0] | hb[1] << 16, hb[2] | hb[3] << 16, hb[4] | hb[5] << 16, hb[6] | hb[7] << 16};
            al[qb][t] = u32x4{lb[0] | lb[1] << 16, lb[2] | lb[3] << 16, lb[4] | lb[5] << 16, lb[6] | lb[7] << 16};
        }
    }
    float lst[FR_QBW][4][FR_J];
#pragma unroll
    for (int qb = 0; qb < FR_QBW; qb++)
#pragma unroll
        for (int r = 0; r < 4; r++)
#pragma unroll
            for (int j = 0; j < FR_J; j++) lst[qb][r][j] = FR_BIG;

    // Stage st: tiles tile0 + FR_TPS st .. + FR_TPS - 1 (chunks contiguous in
    // the packed copy, which is padded to whole groups of four tiles).
    u32x4 pre[PER];
    float pn = 0.0f;
    auto fetch = [&](int st) {
        const size_t base = (size_t)(tile0 + FR_TPS * st) * TC;
#pragma unroll
        for (int i = 0; i < PER; i++) pre[i] = Xb[base + (size_t)i * VGPU_BLOCK + tid];
        const int v = (tile0 + FR_TPS * st) * 16 + tid;
        pn = tid < FR_TPS * 16 && v < n ? Xnorm[v] : 0.0f;
    };
    auto store = [&](int buf) {
#pragma unroll
        for (int i = 0; i < PER; i++) stage[(size_t)buf * SC + i * VGPU_BLOCK + tid] = pre[i];
        if (tid < FR_TPS * 16) snorm[buf * FR_TPS * 16 + tid] = pn;
    };
    // Scores of stage st into the lane's lists: score = base + acc with base
    // ||x||^2 (metric 0) or 1 (the product is -2 q.x or -q.x); only the
    // slice's last stage can hold columns past its tiles or past n.
    auto epilogue = [&](const floatx4 (&acc)[FR_TPS][FR_QBW], const float (&xn)[FR_TPS], int st, bool last) {
#pragma unroll
        for (int i = 0; i < FR_TPS; i++) {
            const int ti = FR_TPS * st + i;  // tile index in the slice, < 2^ib
            const bool colok = !last || (tile0 + ti < tile1 && (tile0 + ti) * 16 + c < n);
            const float base = metric == 0 ? xn[i] : 1.0f;
#pragma unroll
            for (int qb = 0; qb < FR_QBW; qb++)
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    const float v = base + acc[i][qb][r];
                    const float key = __uint_as_float((__float_as_uint(v) & kmask) | (uint32_t)ti);
                    fr_insert(lst[qb][r], colok ? key : FR_BIG);
                }
        }
    };

    floatx4 prev[FR_TPS][FR_QBW];
    float prevn[FR_TPS];
    if (nst > 0) {
        fetch(0);
        store(0);
        if (nst > 1) fetch(1);
    }
    for (int st = 0; st < nst; st++) {
        __syncthreads();  // stage st visible; buffer (st + 1) & 1 no longer read
        if (st + 1 < nst) {
            store((st + 1) & 1);
            if (st + 2 < nst) fetch(st + 2);
        }
        const u32x4* b = stage + (size_t)(st & 1) * SC;
        floatx4 acc[FR_TPS][FR_QBW];
        float xn[FR_TPS];
#pragma unroll
        for (int i = 0; i < FR_TPS; i++) {
            xn[i] = snorm[(st & 1) * FR_TPS * 16 + i * 16 + c];
#pragma unroll
            for (int qb = 0; qb < FR_QBW; qb++) acc[i][qb] = floatx4{0.f, 0.f, 0.f, 0.f};
        }
#pragma unroll
        for (int t = 0; t < DT; t++) {
#pragma unroll
            for (int i = 0; i < FR_TPS; i++) {
                const int o = i * TC + (t * 4 + g) * 16 + c;
                const bf16x8 bh = __builtin_bit_cast(bf16x8, b[o]);
                const bf16x8 bl = __builtin_bit_cast(bf16x8, b[o + DT * 64]);
#pragma unroll
                for (int qb = 0; qb < FR_QBW; qb++) {
                    const bf16x8 a_h = __builtin_bit_cast(bf16x8, ah[qb][t]);
                    const bf16x8 a_l = __builtin_bit_cast(bf16x8, al[qb][t]);
                    acc[i][qb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a_h, bl, acc[i][qb], 0, 0, 0);
                    acc[i][qb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a_l, bh, acc[i][qb], 0, 0, 0);
                    acc[i][qb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a_h, bh, acc[i][qb], 0, 0, 0);
                }
            }
        }
        if (st > 0) epilogue(prev, prevn, st - 1, false);
#pragma unroll
        for (int i = 0; i < FR_TPS; i++) {
            prevn[i] = xn[i];
#pragma unroll
            for (int qb = 0; qb < FR_QBW; qb++) prev[i][qb] = acc[i][qb];
        }
    }
    if (nst > 0) epilogue(prev, prevn, nst - 1, true);

    // Per row: every lane's FR_J keys as (fkey, vector index), ~0 past a
    // short list, and the bound every dropped key is at or above: the
    // FR_J-th key of every full lane list (all 16 FR_J keys are kept, kk =
    // 16 FR_J, so no key of the lists themselves is dropped).
#pragma unroll
    for (int j = 0; j < 4 * FR_QBW; j++) {
        const int qb = j >> 2, r = j & 3;
        const float tl = lst[qb][r][FR_J - 1];
        uint32_t lb = tl < FR_BIG ? fkey(tl) : 0xffffffffu;
#pragma unroll
        for (int o = 1; o < 16; o <<= 1) {
            const uint32_t x = shfl_xor_u32(lb, o);
            lb = x < lb ? x : lb;
        }
        const int qrow = q0 + (FR_QBW * wave + qb) * 16 + 4 * g + r;
        if (qrow < nq) {
            uint64_t* out = partial + ((size_t)qrow * splits + sl) * kk;
#pragma unroll
            for (int e = 0; e < FR_J; e++) {
                const float t = lst[qb][r][e];
                const uint32_t col = (uint32_t)((tile0 + (int)(__float_as_uint(t) & ~kmask)) * 16 + c);
                out[e * 16 + c] = t < FR_BIG ? ((uint64_t)fkey(t) << 32) | col : ~0ull;
            }
            if (c == 0) pbound[(size_t)qrow * splits + sl] = lb;
        }
    }
}

#define FL_BUF 2048
#define FL_ROUND 512

// The reference's distance of query q to row x (rows 16-byte aligned): squared
// L2 or 1 - dot, summed in index order.
__device__ inline float flat_exact(const float* q, const float* __restrict__ x, int d, int metric) {
    return metric == 0 ? seq_l2_stream(q, x, d) : 1.0f - seq_dot_stream(q, x, d);
}

// Exact top-k of query qv over the vectors item(0 .. W - 1) names (an index,
// or 0xffffffff to skip the item) with a threshold-filtered LDS buffer: keys
// (fkey(dist), index) sorted ascending in keys[0 ..) on return; returns how
// many (all threads).  keys / pay hold FL_BUF entries; misc 12 words.
template <class Item>
__device__ int flat_exact_items(const float* qv, const float* __restrict__ X, int W, Item item, int d, int k,
                                int metric, uint64_t* keys, uint32_t* pay, uint32_t* misc) {
    const int tid = threadIdx.x;
    if (tid == 0) {
        misc[2] = 0;
        misc[3] = 0xffffffffu;
    }
    __syncthreads();
    // the buffer count as every thread knows it: each round's appends are
    // counted per wave into misc[4 + 4 par + wave] before the round's barrier
    // and summed after it, so the flush decision is the same in every wave
    // (the shared counter itself may already hold a faster wave's appends)
    uint32_t cnt = 0, par = 0;
    for (int base = 0; base < W; base += FL_ROUND) {
        if ((int)cnt > FL_BUF - FL_ROUND) {
            int m = (int)cnt;
            int m2 = next_pow2(m);
            for (int i = m + tid; i < m2; i += blockDim.x) keys[i] = ~0ull;
            block_bitonic_sort(keys, pay, m2);
            if (tid == 0 && m >= k) {
                misc[3] = (uint32_t)(keys[k - 1] >> 32);
                misc[2] = (uint32_t)k;
            }
            __syncthreads();
            cnt = m >= k ? (uint32_t)k : (uint32_t)m;
        }
        const uint32_t th = misc[3];
        uint32_t wn = 0;
        for (int u = 0; u < FL_ROUND / 256; u++) {
            const int i = base + u * 256 + tid;
            const uint32_t j = i < W ? item(i) : 0xffffffffu;
            bool take = false;
            uint64_t key = 0;
            if (j != 0xffffffffu) {
                key = cand_key(flat_exact(qv, X + (size_t)j * d, d, metric), j);
                take = (uint32_t)(key >> 32) <= th;
            }
            wn += (uint32_t)__popcll(__ballot(take));
            int slot = wave_append_slot(take, &misc[2]);
            if (take) keys[slot] = key;
        }
        if ((tid & 63) == 0) misc[4 + 4 * par + (tid >> 6)] = wn;
        __syncthreads();
        cnt += misc[4 + 4 * par] + misc[5 + 4 * par] + misc[6 + 4 * par] + misc[7 + 4 * par];
        par ^= 1u;
    }
    int m = (int)misc[2];
    int m2 = next_pow2(m > 0 ? m : 1);
    for (int i = m + tid; i < m2; i += blockDim.x) keys[i] = ~0ull;
    block_bitonic_sort(keys, pay, m2);
    return m;
}

// flat_exact_items over vectors [j0, j1).
__device__ int flat_exact_range(const float* qv, const float* __restrict__ X, int j0, int j1, int d, int k,
                                int metric, uint64_t* keys, uint32_t* pay, uint32_t* misc) {
    return flat_exact_items(qv, X, j1 > j0 ? j1 - j0 : 0, [=](int i) { return (uint32_t)(j0 + i); }, d, k,
                            metric, keys, pay, misc);
}

__global__ __launch_bounds__(256) void flat_merge_kernel(
    const uint64_t* __restrict__ partial, int splits, int kk, const float* __restrict__ Q,
    const float* __restrict__ Qsq, const float* __restrict__ X, int nq, int n, int d, int k,
    int metric, float xmax, const uint32_t* __restrict__ pbound, int ib, uint32_t* __restrict__ out_idx,
    float* __restrict__ out_dist, unsigned int* overflow, uint32_t* __restrict__ flag_list) {
    __shared__ uint64_t keys[FL_BUF];
    __shared__ uint32_t pay[FL_BUF];
    __shared__ uint32_t misc[12];
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
    // Proof.  A_k = the k-th smallest kept ranking key; the k kept entries with
    // the smallest keys have exact distances <= A_k + tau, so every member of
    // the exact top-k has a key <= bound = A_k + 2 tau.  An entry a slice
    // dropped has a key >= that slice's bound (pbound, or its kk-th kept key)
    // >= B, the smallest over the slices.  B > bound: the kept entries with
    // keys <= bound hold the exact top-k (ties included), and they are
    // rescored.  Fewer than k kept entries: every slice kept all it saw.
    if (tid == 0) {
        int m = 0, hi = tot;  // valid keys (the ~0 padding sorts last)
        while (m < hi) {
            const int mid = (m + hi) >> 1;
            if (keys[mid] != ~0ull) m = mid + 1;
            else hi = mid;
        }
        uint32_t fail = 0, rescore = (uint32_t)m;
        if (m >= k) {
            const float u = 5.9604645e-08f;
            const float qmax = sqrtf(Qsq[q]) * 1.0001f + 1e-30f;
            const float tau = pbound ? flat_bf16_tau(d, metric, qmax, xmax, ib)
                                     : metric == 0 ? 4.0f * (float)(d + 8) * u * (qmax + xmax) * (qmax + xmax)
                                                   : 4.0f * (float)(d + 8) * u * (1.0f + qmax * xmax);
            uint32_t fb = fkey(key_dist(keys[k - 1]) + 2.0f * tau);
            fb = fb < 0xfffffffeu ? fb + 1u : 0xffffffffu;  // one ulp up: the bound is not rounded down
            uint32_t B = 0xffffffffu;
            for (int sl = 0; sl < splits; sl++) {
                uint32_t b = 0xffffffffu;
                if (pbound) {
                    b = pbound[(size_t)q * splits + sl];
                } else {
                    const uint64_t last = partial[((size_t)q * splits + sl) * kk + kk - 1];
                    if (last != ~0ull) b = (uint32_t)(last >> 32);
                }
                B = b < B ? b : B;
            }
            if (!(B > fb)) {
                fail = 1;
            } else {
                int lo = 0;
                hi = m;  // keys whose high word is <= fb
                while (lo < hi) {
                    const int mid = (lo + hi) >> 1;
                    if ((uint32_t)(keys[mid] >> 32) <= fb) lo = mid + 1;
                    else hi = mid;
                }
                rescore = (uint32_t)lo;
            }
        }
        misc[0] = rescore;
        misc[1] = fail;
        // an unproved query is answered by the exhaustive exact scan, spread
        // over many workgroups by launch_flat_fallback
        if (fail) flag_list[atomicAdd(overflow, 1u)] = (uint32_t)q;
    }
    __syncthreads();
    const int have = (int)misc[0];
    if (misc[1]) return;
    {
        for (int i = tid; i < n2; i += blockDim.x) {
            if (i < have) {
                uint32_t idx = (uint32_t)keys[i];
                keys[i] = cand_key(flat_exact(qv, X + (size_t)idx * d, d, metric), idx);
            } else {
                keys[i] = ~0ull;
            }
        }
        block_bitonic_sort(keys, pay, n2);
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

// Merge of the ranking kernel's slices, one wave per query (four per
// workgroup), keys in registers: key i = e * 64 + lane in k[e].  The proof is
// flat_merge_kernel's: A_k by a bitwise search over the keys' high words
// (ballot counts), B the smallest slice bound; the keys <= A_k + 2 tau (at
// most FM_R) are compacted through LDS, rescored with the reference's
// arithmetic and sorted in registers.  More than FM_R such keys, or no
// proof: the query goes to the exhaustive fallback.
#define FM_R 256
template <int E>
__global__ __launch_bounds__(256) void flat_merge_wave_kernel(
    const uint64_t* __restrict__ partial, const uint32_t* __restrict__ pbound, int splits, int kk,
    const float* __restrict__ Q, const float* __restrict__ Qsq, const float* __restrict__ X, int nq, int d,
    int k, int metric, float xmax, int ib, uint32_t* __restrict__ out_idx, float* __restrict__ out_dist,
    unsigned int* overflow, uint32_t* __restrict__ flag_list, uint32_t* __restrict__ fbv) {
    __shared__ uint64_t rbuf[4][FM_R];
    __shared__ float qsh[4][128];  // d <= 128
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int q = blockIdx.x * 4 + wave;
    if (q >= nq) return;
    // the query to LDS (rescoring) and, without Qsq, its squared norm for the
    // error bound (any order: the bound takes sqrt(.) * 1.0001)
    const float* qv = qsh[wave];
    float qsq = 0.0f;
    for (int j = lane; j < d; j += 64) {
        const float x = Q[(size_t)q * d + j];
        qsh[wave][j] = x;
        qsq = __builtin_fmaf(x, x, qsq);
    }
    if (Qsq) {
        qsq = Qsq[q];
    } else {
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) qsq += __uint_as_float(shfl_xor_u32(__float_as_uint(qsq), o));
    }
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
    __builtin_amdgcn_wave_barrier();
    const int tot = splits * kk;
    uint64_t kv[E];
    const uint64_t* src = partial + (size_t)q * tot;
#pragma unroll
    for (int e = 0; e < E; e++) {
        const int i = e * 64 + lane;
        kv[e] = i < tot ? src[i] : ~0ull;
    }
    int m = 0;  // valid keys (padding is ~0)
#pragma unroll
    for (int e = 0; e < E; e++) m += (int)__popcll(__ballot(kv[e] != ~0ull));
    uint32_t fb = 0xffffffffu;  // keys whose high word is <= fb are rescored
    if (m >= k) {
        uint32_t T = 0;  // the (k-1)-th smallest high word: the largest v with < k words below it
        for (int b = 31; b >= 0; b--) {
            const uint32_t cand = T | (1u << b);
            int below = 0;
#pragma unroll
            for (int e = 0; e < E; e++) below += (int)__popcll(__ballot((uint32_t)(kv[e] >> 32) < cand));
            if (below <= k - 1) T = cand;
        }
        const float u = 5.9604645e-08f;
        const float qmax = sqrtf(qsq) * 1.0001f + 1e-30f;
        const float tau = flat_bf16_tau(d, metric, qmax, xmax, ib);
        fb = fkey(fkey_to_float(T) + 2.0f * tau);
        fb = fb < 0xfffffffeu ? fb + 1u : 0xffffffffu;  // one ulp up: the bound is not rounded down
        (void)u;
        uint32_t B = 0xffffffffu;
        for (int sl = lane; sl < splits; sl += 64) {
            const uint32_t b = pbound[(size_t)q * splits + sl];
            B = b < B ? b : B;
        }
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) {
            const uint32_t x = (uint32_t)__shfl_xor((int)B, o, 64);
            B = x < B ? x : B;
        }
        if (!(B > fb)) {
            if (lane == 0) {
                fbv[q] = fb;
                flag_list[atomicAdd(overflow, 1u)] = (uint32_t)q;
            }
            return;
        }
    }
    // compact the keys <= fb into this wave's LDS row
    uint32_t cnt = 0;
#pragma unroll
    for (int e = 0; e < E; e++) {
        const bool take = kv[e] != ~0ull && (uint32_t)(kv[e] >> 32) <= fb;
        const uint64_t mk = __ballot(take);
        const uint32_t pos = cnt + __builtin_amdgcn_mbcnt_hi((uint32_t)(mk >> 32),
                                                             __builtin_amdgcn_mbcnt_lo((uint32_t)mk, 0u));
        if (take && pos < FM_R) rbuf[wave][pos] = kv[e];
        cnt += (uint32_t)__popcll(mk);
    }
    if (cnt > FM_R) {  // more near-ties than the rescoring holds
        if (lane == 0) {
            fbv[q] = fb;
            flag_list[atomicAdd(overflow, 1u)] = (uint32_t)q;
        }
        return;
    }
    auto rescore = [&](uint32_t i) -> uint64_t {
        if (i >= cnt) return ~0ull;
        const uint32_t idx = (uint32_t)rbuf[wave][i];
        return cand_key(flat_exact(qv, X + (size_t)idx * d, d, metric), idx);
    };
    auto emit = [&](int j, uint64_t key) {
        if (j < k) {
            const size_t o = (size_t)q * k + j;
            out_idx[o] = key != ~0ull ? (uint32_t)key : 0xffffffffu;
            out_dist[o] = key != ~0ull ? key_dist(key) : __int_as_float(0x7f800000);
        }
    };
    if (cnt <= 64) {  // the usual case: one key per lane
        uint64_t r1[1] = {rescore((uint32_t)lane)};
        wave_sort_regs<1>(r1);
        emit(lane, r1[0]);
        return;
    }
    uint64_t r[FM_R / 64];
#pragma unroll
    for (int e = 0; e < FM_R / 64; e++) r[e] = rescore((uint32_t)(e * 64 + lane));
    wave_sort_regs<FM_R / 64>(r);
#pragma unroll
    for (int e = 0; e < FM_R / 64; e++) emit(e * 64 + lane, r[e]);
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

// The bf16x3 ranking kernel serves d <= 128 and k <= 32; every slice keeps
// all 16 FR_J keys of a row's lane lists, plus one bound word per (query,
// slice) after the keys.
static bool flat_rank_ok(int d, int k) { return d >= 1 && d <= 128 && k >= 1 && k <= 32; }
static int flat_rank_keep(int k) {
    (void)k;
    return 16 * FR_J;
}

// Slices for the ranking kernel: a whole number of stages (FR_TPS tiles)
// each, enough workgroups for four waves of two per CU on 256 CUs, slices of
// at least 64 tiles, and splits * kk merge entries within the merge buffer;
// ib = the bits of a tile index within a slice.
static int flat_rank_splits(int nq, int n, int kk, int* tps, int* ib) {
    const int qb = (nq + FR_ROWS - 1) / FR_ROWS, ntiles = (n + 15) / 16;
    int sp = 1;
    while (qb * sp < 2048 && 2 * sp * kk <= FL_BUF && ntiles / (2 * sp) >= 64) sp <<= 1;
    int t = (ntiles + sp - 1) / sp;
    t = (t + FR_TPS - 1) / FR_TPS * FR_TPS;  // whole stages: a stage never reaches past the padded copy
    int b = 1;
    while ((1 << b) < t) b++;
    *tps = t;
    *ib = b;
    return (ntiles + t - 1) / t;
}

// Exhaustive exact fallback of the unproved queries, spread over the GPU:
// workgroup (s, i) finds the exact top-k of query flag_list[i] among vectors
// [s len, (s + 1) len) and writes its k smallest keys (padded with ~0); the
// finish kernel merges a query's slices and writes its output row.
__global__ __launch_bounds__(256) void flat_exact_slice_kernel(
    const uint32_t* __restrict__ flag_list, const float* __restrict__ Q, const float* __restrict__ X, int n,
    int d, int k, int metric, int len, uint64_t* __restrict__ out_keys) {
    __shared__ uint64_t keys[FL_BUF];
    __shared__ uint32_t pay[FL_BUF];
    __shared__ uint32_t misc[12];
    const int s = blockIdx.x, i = blockIdx.y, tid = threadIdx.x;
    const uint32_t q = flag_list[i];
    const int j0 = s * len, j1 = min(n, j0 + len);
    const int m = flat_exact_range(Q + (size_t)q * d, X, j0, j1, d, k, metric, keys, pay, misc);
    for (int j = tid; j < k; j += blockDim.x)
        out_keys[((size_t)i * gridDim.x + s) * k + j] = j < m ? keys[j] : ~0ull;
}

// nflag_dev (optional): the flagged-query count on the device; workgroups
// past it (or past the grid) have nothing to do.
__global__ __launch_bounds__(256) void flat_exact_finish_kernel(
    const uint32_t* __restrict__ flag_list, int slices, int k, const uint64_t* __restrict__ in_keys,
    uint32_t* __restrict__ out_idx, float* __restrict__ out_dist, const unsigned int* nflag_dev) {
    __shared__ uint64_t keys[FL_BUF];
    __shared__ uint32_t pay[FL_BUF];
    const int i = blockIdx.x, tid = threadIdx.x;
    if (nflag_dev && (unsigned int)i >= *nflag_dev) return;
    const uint32_t q = flag_list[i];
    const int tot = slices * k, n2 = next_pow2(tot);
    for (int j = tid; j < n2; j += blockDim.x) {
        keys[j] = j < tot ? in_keys[(size_t)i * tot + j] : ~0ull;
        pay[j] = 0;
    }
    block_bitonic_sort(keys, pay, n2);
    for (int j = tid; j < k; j += blockDim.x) {
        const size_t o = (size_t)q * k + j;
        const uint64_t key = keys[j];
        out_idx[o] = key != ~0ull ? (uint32_t)key : 0xffffffffu;
        out_dist[o] = key != ~0ull ? key_dist(key) : __int_as_float(0x7f800000);
    }
}

// Fallback of the ranking path, workgroup (s, i) for query q = flag_list[i]
// and ranking slice s (tiles s tps ..), fb = the query's rescoring threshold
// fbv[q].  Lane c of a slice's row kept the FR_J smallest keys of vectors
// 16 (s tps + t) + c (t < tps) at partial[e 16 + c], sorted in e; a lane whose
// list is not full dropped nothing, and one whose FR_J-th key exceeds fb
// dropped no key <= fb.  The other lanes' columns are scanned with the exact
// arithmetic, and the kept keys <= fb of the rest are rescored: every vector
// with a key <= fb (the superset of the exact top-k the merge proved) is
// scored exactly, so the slice's k smallest exact keys, written to out_keys
// for flat_exact_finish_kernel, hold its share of the exact top-k.
__global__ __launch_bounds__(256) void flat_rank_fallback_kernel(
    const uint32_t* __restrict__ flag_list, const uint32_t* __restrict__ fbv,
    const uint64_t* __restrict__ partial, const uint32_t* __restrict__ pbound, int splits, int kk, int tps,
    const float* __restrict__ Q, const float* __restrict__ X, int n, int d, int k, int metric,
    uint64_t* __restrict__ out_keys, const unsigned int* nflag_dev) {
    if (nflag_dev && blockIdx.y >= *nflag_dev) return;  // uniform: no flagged query for this row
    __shared__ uint64_t keys[FL_BUF];
    __shared__ uint32_t pay[FL_BUF];
    __shared__ uint32_t misc[12];
    __shared__ float qs[128];  // d <= 128
    __shared__ uint32_t rescan[16];
    const int s = blockIdx.x, i = blockIdx.y, tid = threadIdx.x;
    const uint32_t q = flag_list[i];
    const uint32_t fb = fbv[q];
    const uint64_t* src = partial + ((size_t)q * splits + s) * kk;
    uint64_t* out = out_keys + ((size_t)i * splits + s) * k;
    for (int j = tid; j < d; j += blockDim.x) qs[j] = Q[(size_t)q * d + j];
    __syncthreads();
    if (pbound[(size_t)q * splits + s] > fb) {
        if (tid >= 64) return;  // kk <= 64 kept keys: one wave
        uint64_t r[1] = {~0ull};
        if (tid < kk) {
            const uint64_t key = src[tid];
            if (key != ~0ull && (uint32_t)(key >> 32) <= fb) {
                const uint32_t idx = (uint32_t)key;
                r[0] = cand_key(flat_exact(qs, X + (size_t)idx * d, d, metric), idx);
            }
        }
        wave_sort_regs<1>(r);
        if (tid < k) out[tid] = r[0];
        return;
    }
    // the lanes to rescan: full list (FR_J-th key present) with that key <= fb
    uint32_t nres = 0, resmask = 0;
    for (int c = 0; c < 16; c++) {
        const uint64_t last = src[(FR_J - 1) * 16 + c];
        if (last != ~0ull && (uint32_t)(last >> 32) <= fb) {
            if (tid == 0) rescan[nres] = (uint32_t)c;
            nres++;
            resmask |= 1u << c;
        }
    }
    __syncthreads();
    const int scan = (int)nres * tps, tile0 = s * tps;
    auto item = [&](int it) -> uint32_t {
        if (it < scan) {
            const int t = it % tps;
            const uint32_t v = (uint32_t)((tile0 + t) * 16) + rescan[it / tps];
            return v < (uint32_t)n ? v : 0xffffffffu;
        }
        const uint64_t key = src[it - scan];
        const bool kept = key != ~0ull && (uint32_t)(key >> 32) <= fb && !((resmask >> ((it - scan) & 15)) & 1u);
        return kept ? (uint32_t)key : 0xffffffffu;
    };
    const int m = flat_exact_items(qs, X, scan + kk, item, d, k, metric, keys, pay, misc);
    for (int j = tid; j < k; j += blockDim.x) out[j] = j < m ? keys[j] : ~0ull;
}

int flat_fallback_slices(int n, int k) {
    int sl = FL_BUF / k;
    sl = sl > 256 ? 256 : sl;
    const int most = (n + 255) / 256;  // at least 256 vectors per slice
    return sl < most ? sl : (most > 0 ? most : 1);
}

void launch_flat_rank_fallback(const uint32_t* flag_list, int nflag, const uint32_t* fbv,
                               const uint64_t* partial, int nq, int n, int d, int k, int metric,
                               const float* Q, const float* X, uint64_t* keys, uint32_t* out_idx,
                               float* out_dist, hipStream_t s) {
    int tps, ib;
    const int kk = flat_rank_keep(k), sp = flat_rank_splits(nq, n, kk, &tps, &ib);
    const uint32_t* pbound = reinterpret_cast<const uint32_t*>(partial + (size_t)nq * sp * kk);
    for (int f0 = 0; f0 < nflag; f0 += 65535) {  // grid.y limit
        const int nf = nflag - f0 < 65535 ? nflag - f0 : 65535;
        hipLaunchKernelGGL(flat_rank_fallback_kernel, dim3(sp, nf), dim3(256), 0, s, flag_list + f0, fbv, partial,
                           pbound, sp, kk, tps, Q, X, n, d, k, metric, keys + (size_t)f0 * sp * k, nullptr);
        hipLaunchKernelGGL(flat_exact_finish_kernel, dim3(nf), dim3(256), 0, s, flag_list + f0, sp, k,
                           keys + (size_t)f0 * sp * k, out_idx, out_dist, nullptr);
    }
}

void launch_flat_rank_fallback_dev(const uint32_t* flag_list, const unsigned int* nflag_dev, int cap,
                                   const uint32_t* fbv, const uint64_t* partial, int nq, int n, int d, int k,
                                   int metric, const float* Q, const float* X, uint64_t* keys, uint32_t* out_idx,
                                   float* out_dist, hipStream_t s) {
    if (cap <= 0) return;
    int tps, ib;
    const int kk = flat_rank_keep(k), sp = flat_rank_splits(nq, n, kk, &tps, &ib);
    const uint32_t* pbound = reinterpret_cast<const uint32_t*>(partial + (size_t)nq * sp * kk);
    hipLaunchKernelGGL(flat_rank_fallback_kernel, dim3(sp, cap), dim3(256), 0, s, flag_list, fbv, partial, pbound,
                       sp, kk, tps, Q, X, n, d, k, metric, keys, nflag_dev);
    hipLaunchKernelGGL(flat_exact_finish_kernel, dim3(cap), dim3(256), 0, s, flag_list, sp, k, keys, out_idx,
                       out_dist, nflag_dev);
}

int flat_rank_fallback_slices(int nq, int n, int d, int k) {
    if (!flat_rank_ok(d, k)) return 0;
    int tps, ib;
    return flat_rank_splits(nq, n, flat_rank_keep(k), &tps, &ib);
}

void launch_flat_fallback(const uint32_t* flag_list, int nflag, const float* Q, const float* X, int n, int d,
                          int k, int metric, uint64_t* keys, uint32_t* out_idx, float* out_dist,
                          hipStream_t s) {
    const int sl = flat_fallback_slices(n, k), len = (n + sl - 1) / sl;
    for (int f0 = 0; f0 < nflag; f0 += 65535) {  // grid.y limit
        const int nf = nflag - f0 < 65535 ? nflag - f0 : 65535;
        hipLaunchKernelGGL(flat_exact_slice_kernel, dim3(sl, nf), dim3(256), 0, s, flag_list + f0, Q, X, n, d,
                           k, metric, len, keys + (size_t)f0 * sl * k);
        hipLaunchKernelGGL(flat_exact_finish_kernel, dim3(nf), dim3(256), 0, s, flag_list + f0, sl, k,
                           keys + (size_t)f0 * sl * k, out_idx, out_dist, nullptr);
    }
}


size_t flat_partial_count(int nq, int n, int d, int k) {
    if (flat_rank_ok(d, k)) {
        int tps, ib;
        const int kk = flat_rank_keep(k);
        const size_t slots = (size_t)nq * flat_rank_splits(nq, n, kk, &tps, &ib);
        return slots * kk + (slots + 1) / 2;
    }
    return (size_t)nq * flat_splits(nq, n, flat_keep(k)) * flat_keep(k);
}

size_t flat_pack_chunks(int n, int d) { return d <= 128 ? coarse_bf16_pack_chunks(n, d) : 0; }

void launch_flat_pack(const float* X, int n, int d, uint4* Xb, hipStream_t s) {
    if (d <= 128 && n > 0) launch_coarse_bf16_pack(X, n, d, Xb, s);
}

template <int DT>
static void launch_rank(const float* Q, int nq, int d, const uint4* Xb, const float* Xnorm, int n, int metric,
                        int kk, int tps, int ib, int sp, uint64_t* partial, uint32_t* pbound, hipStream_t s) {
    const size_t lds = 2 * (size_t)FR_TPS * 2 * DT * 64 * 16 + 2 * FR_TPS * 16 * 4;
    ensure_dyn_lds((const void*)flat_rank_kernel<DT>, lds);
    dim3 grid((nq + FR_ROWS - 1) / FR_ROWS, sp);
    hipLaunchKernelGGL(flat_rank_kernel<DT>, grid, dim3(VGPU_BLOCK), lds, s, Q, nq, d, Xb, Xnorm, n, metric, kk,
                       tps, ib, sp, partial, pbound);
}

void launch_flat_search(const float* Q, const float* Qsq, int nq, const float* X, const uint4* Xb,
                        const float* Xnorm, int n, int d, int k, int metric, float xmax,
                        uint64_t* partial, uint32_t* out_idx, float* out_dist,
                        unsigned int* overflow, uint32_t* flag_list, uint32_t* fbv, hipStream_t s,
                        hipEvent_t ranked) {
    if (nq <= 0) return;
    if (Xb && flat_rank_ok(d, k)) {
        int tps, ib;
        const int kk = flat_rank_keep(k), sp = flat_rank_splits(nq, n, kk, &tps, &ib);
        uint32_t* pbound = reinterpret_cast<uint32_t*>(partial + (size_t)nq * sp * kk);
        switch ((d + 31) / 32) {
            case 1: launch_rank<1>(Q, nq, d, Xb, Xnorm, n, metric, kk, tps, ib, sp, partial, pbound, s); break;
            case 2: launch_rank<2>(Q, nq, d, Xb, Xnorm, n, metric, kk, tps, ib, sp, partial, pbound, s); break;
            case 3: launch_rank<3>(Q, nq, d, Xb, Xnorm, n, metric, kk, tps, ib, sp, partial, pbound, s); break;
            default: launch_rank<4>(Q, nq, d, Xb, Xnorm, n, metric, kk, tps, ib, sp, partial, pbound, s); break;
        }
        if (ranked) (void)hipEventRecord(ranked, s);
        const int tot = sp * kk;
        const dim3 mg((nq + 3) / 4);
        if (tot <= 256)
            hipLaunchKernelGGL(flat_merge_wave_kernel<4>, mg, dim3(256), 0, s, partial, pbound, sp, kk, Q, Qsq, X,
                               nq, d, k, metric, xmax, ib, out_idx, out_dist, overflow, flag_list, fbv);
        else if (tot <= 512)
            hipLaunchKernelGGL(flat_merge_wave_kernel<8>, mg, dim3(256), 0, s, partial, pbound, sp, kk, Q, Qsq, X,
                               nq, d, k, metric, xmax, ib, out_idx, out_dist, overflow, flag_list, fbv);
        else if (tot <= 1024)
            hipLaunchKernelGGL(flat_merge_wave_kernel<16>, mg, dim3(256), 0, s, partial, pbound, sp, kk, Q, Qsq,
                               X, nq, d, k, metric, xmax, ib, out_idx, out_dist, overflow, flag_list, fbv);
        else
            hipLaunchKernelGGL(flat_merge_wave_kernel<32>, mg, dim3(256), 0, s, partial, pbound, sp, kk, Q, Qsq,
                               X, nq, d, k, metric, xmax, ib, out_idx, out_dist, overflow, flag_list, fbv);
        return;
    }
    const int kk = flat_keep(k), cap = flat_cap(kk), sp = flat_splits(nq, n, kk);
    const int chunk = (((n + sp - 1) / sp) + FL_N - 1) / FL_N * FL_N;
    size_t lds = 2 * FL_Q * (FL_K + 1) * 4 + (size_t)FL_Q * cap * 8 + 2 * FL_Q * 4;
    ensure_dyn_lds((const void*)flat_partial_kernel, lds);
    dim3 grid((nq + FL_Q - 1) / FL_Q, sp);
    hipLaunchKernelGGL(flat_partial_kernel, grid, dim3(256), lds, s, Q, X, Xnorm, nq, n, d, metric, kk,
                       cap, sp, chunk, partial);
    if (ranked) (void)hipEventRecord(ranked, s);
    hipLaunchKernelGGL(flat_merge_kernel, dim3(nq), dim3(256), 0, s, partial, sp, kk, Q, Qsq, X, nq, n,
                       d, k, metric, xmax, nullptr, 0, out_idx, out_dist, overflow, flag_list);
}

}  // namespace vgpu
