// Device helpers shared by the gfx950 kernels: total-order float keys, a
// block-wide bitonic sort in LDS, a block-wide radix select and wave-level
// append for top-k buffers.  The block-wide helpers assume 256 threads (4
// waves of 64), the launch shape of every kernel that calls them.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#define VGPU_BLOCK 256
#define VGPU_WAVE 64

// True when one of the n values is a NaN or an infinity (exponent all ones).
__device__ __forceinline__ bool row_nonfinite(const float* x, int n) {
    uint32_t any = 0;
    for (int j = 0; j < n; j++) any |= (__float_as_uint(x[j]) & 0x7f800000u) == 0x7f800000u;
    return any != 0;
}

// f32::total_cmp as an unsigned key: u32 order == total_cmp order
// (src/ivf_pq/search.rs:64-75 sorts with total_cmp; NaN sorts last).
__device__ __forceinline__ uint32_t fkey(float f) {
    uint32_t b = __float_as_uint(f);
    return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}

__device__ __forceinline__ float fkey_to_float(uint32_t k) {
    uint32_t b = (k & 0x80000000u) ? (k & 0x7fffffffu) : ~k;
    return __uint_as_float(b);
}

// Candidate key: distance in the high word, vector index in the low word, so
// u64 order = (distance total_cmp, then lower vector index).
__device__ __forceinline__ uint64_t cand_key(float dist, uint32_t idx) {
    return ((uint64_t)fkey(dist) << 32) | idx;
}

__device__ __forceinline__ float key_dist(uint64_t key) { return fkey_to_float((uint32_t)(key >> 32)); }

// Sequential float32 dot product (src/simd.rs:88-91 order); the library is
// compiled with -ffp-contract=off so each step rounds the product and the sum.
__device__ __forceinline__ float seq_dot(const float* a, const float* b, int n) {
    float s = 0.0f;
    for (int i = 0; i < n; i++) s += a[i] * b[i];
    return s;
}

// The same sequential order with the second operand streamed from global
// memory 32 floats at a time (eight 16-byte loads in flight per step), for
// d % 4 == 0 and 16-byte aligned b; other shapes take seq_dot.
__device__ __forceinline__ float seq_dot_stream(const float* a, const float* __restrict__ b, int d) {
    if ((d & 3) != 0) return seq_dot(a, b, d);
    float s = 0.0f;
    int j0 = 0;
    for (; j0 + 32 <= d; j0 += 32) {
        float4 v[8];
#pragma unroll
        for (int i = 0; i < 8; i++) v[i] = reinterpret_cast<const float4*>(b + j0)[i];
#pragma unroll
        for (int i = 0; i < 8; i++) {
            s = __fadd_rn(s, __fmul_rn(a[j0 + 4 * i], v[i].x));
            s = __fadd_rn(s, __fmul_rn(a[j0 + 4 * i + 1], v[i].y));
            s = __fadd_rn(s, __fmul_rn(a[j0 + 4 * i + 2], v[i].z));
            s = __fadd_rn(s, __fmul_rn(a[j0 + 4 * i + 3], v[i].w));
        }
    }
    for (; j0 < d; j0 += 4) {
        const float4 v = reinterpret_cast<const float4*>(b + j0)[0];
        s = __fadd_rn(s, __fmul_rn(a[j0], v.x));
        s = __fadd_rn(s, __fmul_rn(a[j0 + 1], v.y));
        s = __fadd_rn(s, __fmul_rn(a[j0 + 2], v.z));
        s = __fadd_rn(s, __fmul_rn(a[j0 + 3], v.w));
    }
    return s;
}

// sum_j (a_j - b_j)^2 in index order, each difference, square and sum
// rounded (the reference's squared-L2 loop), b streamed as seq_dot_stream
// streams it; d % 4 == 0 and 16-byte aligned b, other shapes one float at a time.
__device__ __forceinline__ float seq_l2_stream(const float* a, const float* __restrict__ b, int d) {
    float s = 0.0f;
    int j0 = 0;
    if ((d & 3) == 0) {
        for (; j0 + 32 <= d; j0 += 32) {
            float4 v[8];
#pragma unroll
            for (int i = 0; i < 8; i++) v[i] = reinterpret_cast<const float4*>(b + j0)[i];
#pragma unroll
            for (int i = 0; i < 8; i++) {
                const float t0 = __fsub_rn(a[j0 + 4 * i], v[i].x), t1 = __fsub_rn(a[j0 + 4 * i + 1], v[i].y);
                const float t2 = __fsub_rn(a[j0 + 4 * i + 2], v[i].z), t3 = __fsub_rn(a[j0 + 4 * i + 3], v[i].w);
                s = __fadd_rn(s, __fmul_rn(t0, t0));
                s = __fadd_rn(s, __fmul_rn(t1, t1));
                s = __fadd_rn(s, __fmul_rn(t2, t2));
                s = __fadd_rn(s, __fmul_rn(t3, t3));
            }
        }
        for (; j0 < d; j0 += 4) {
            const float4 v = reinterpret_cast<const float4*>(b + j0)[0];
            const float t0 = __fsub_rn(a[j0], v.x), t1 = __fsub_rn(a[j0 + 1], v.y);
            const float t2 = __fsub_rn(a[j0 + 2], v.z), t3 = __fsub_rn(a[j0 + 3], v.w);
            s = __fadd_rn(s, __fmul_rn(t0, t0));
            s = __fadd_rn(s, __fmul_rn(t1, t1));
            s = __fadd_rn(s, __fmul_rn(t2, t2));
            s = __fadd_rn(s, __fmul_rn(t3, t3));
        }
    }
    for (; j0 < d; j0++) {
        const float t = __fsub_rn(a[j0], b[j0]);
        s = __fadd_rn(s, __fmul_rn(t, t));
    }
    return s;
}

// a . b in any order: fused multiply-adds into four partial sums, for ranking
// only.  Within (d / 4 + 2) u sum|a_j b_j| of the real product (u = 2^-24).
// b is 16-byte aligned when d % 4 == 0.
__device__ __forceinline__ float approx_dot(const float* a, const float* __restrict__ b, int d) {
    float s0 = 0.0f, s1 = 0.0f, s2 = 0.0f, s3 = 0.0f;
    int j = 0;
    if ((d & 3) == 0) {
        for (; j + 16 <= d; j += 16) {
            float4 v[4];
#pragma unroll
            for (int i = 0; i < 4; i++) v[i] = reinterpret_cast<const float4*>(b + j)[i];
#pragma unroll
            for (int i = 0; i < 4; i++) {
                s0 = fmaf(a[j + 4 * i], v[i].x, s0);
                s1 = fmaf(a[j + 4 * i + 1], v[i].y, s1);
                s2 = fmaf(a[j + 4 * i + 2], v[i].z, s2);
                s3 = fmaf(a[j + 4 * i + 3], v[i].w, s3);
            }
        }
    }
    for (; j < d; j++) s0 = fmaf(a[j], b[j], s0);
    return (s0 + s1) + (s2 + s3);
}

// approx_dot of a against NR rows b_r = b + r * rs (r < NR) at once, for
// d % 32 == 0 and 16-byte aligned rows: 8 loads of each row in flight per
// step.  Same per-row bound as approx_dot.
template <int NR>
__device__ __forceinline__ void approx_dot_rows(const float* a, const float* __restrict__ b, size_t rs,
                                                int d, float (&out)[NR]) {
    float s[NR][4];
#pragma unroll
    for (int r = 0; r < NR; r++) s[r][0] = s[r][1] = s[r][2] = s[r][3] = 0.0f;
    for (int j = 0; j < d; j += 32) {
        float4 v[NR][8];
#pragma unroll
        for (int r = 0; r < NR; r++)
#pragma unroll
            for (int i = 0; i < 8; i++) v[r][i] = reinterpret_cast<const float4*>(b + r * rs + j)[i];
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const float4 q = *reinterpret_cast<const float4*>(a + j + 4 * i);
#pragma unroll
            for (int r = 0; r < NR; r++) {
                s[r][0] = fmaf(q.x, v[r][i].x, s[r][0]);
                s[r][1] = fmaf(q.y, v[r][i].y, s[r][1]);
                s[r][2] = fmaf(q.z, v[r][i].z, s[r][2]);
                s[r][3] = fmaf(q.w, v[r][i].w, s[r][3]);
            }
        }
    }
#pragma unroll
    for (int r = 0; r < NR; r++) out[r] = (s[r][0] + s[r][1]) + (s[r][2] + s[r][3]);
}

// Ascending bitonic sort of keys[0..n) (n a power of two) with a payload array.
// All threads of the block must call it.
template <typename P>
__device__ void block_bitonic_sort(uint64_t* keys, P* pay, int n) {
    for (int size = 2; size <= n; size <<= 1) {
        for (int stride = size >> 1; stride > 0; stride >>= 1) {
            __syncthreads();
            for (int t = threadIdx.x; t < (n >> 1); t += VGPU_BLOCK) {
                int i = 2 * t - (t & (stride - 1));
                int j = i + stride;
                bool asc = (i & size) == 0;
                uint64_t a = keys[i], b = keys[j];
                if ((a > b) == asc) {
                    keys[i] = b;
                    keys[j] = a;
                    P pa = pay[i];
                    pay[i] = pay[j];
                    pay[j] = pa;
                }
            }
        }
    }
    __syncthreads();
}

// Two payload arrays.
template <typename P, typename Q>
__device__ void block_bitonic_sort2(uint64_t* keys, P* pay, Q* pay2, int n) {
    for (int size = 2; size <= n; size <<= 1) {
        for (int stride = size >> 1; stride > 0; stride >>= 1) {
            __syncthreads();
            for (int t = threadIdx.x; t < (n >> 1); t += blockDim.x) {
                int i = 2 * t - (t & (stride - 1));
                int j = i + stride;
                bool asc = (i & size) == 0;
                uint64_t a = keys[i], b = keys[j];
                if ((a > b) == asc) {
                    keys[i] = b;
                    keys[j] = a;
                    P pa = pay[i];
                    pay[i] = pay[j];
                    pay[j] = pa;
                    Q qa = pay2[i];
                    pay2[i] = pay2[j];
                    pay2[j] = qa;
                }
            }
        }
    }
    __syncthreads();
}

// Ascending bitonic sort of keys[0..n) (n a power of two), keys only.
__device__ inline void block_bitonic_sort_keys(uint64_t* keys, int n) {
    for (int size = 2; size <= n; size <<= 1) {
        for (int stride = size >> 1; stride > 0; stride >>= 1) {
            __syncthreads();
            for (int t = threadIdx.x; t < (n >> 1); t += VGPU_BLOCK) {
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
    __syncthreads();
}

__device__ __forceinline__ int next_pow2(int n) {
    int p = 1;
    while (p < n) p <<= 1;
    return p;
}

// Shared scratch of the radix select: 256 histogram bins + 2 result words.
struct RadixScratch {
    uint32_t hist[256];
    uint32_t bin;
    uint32_t rem;
};

// Block-wide radix select: returns the key of 0-based rank `rank` among the
// keys produced by key_of(i), i in [0, n).  KeyT is uint32_t or uint64_t;
// digits are 8 bits, most significant first.  key_of is called once per
// element per pass.  All threads must call it; rank < n.
template <typename KeyT, typename KeyFn>
__device__ KeyT block_radix_select(KeyFn key_of, int n, uint32_t rank, RadixScratch* rs) {
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    KeyT prefix = 0, mask = 0;
    for (int shift = (int)(sizeof(KeyT) * 8) - 8; shift >= 0; shift -= 8) {
        __syncthreads();
        for (int i = tid; i < 256; i += VGPU_BLOCK) rs->hist[i] = 0;
        __syncthreads();
        for (int i = tid; i < n; i += VGPU_BLOCK) {
            KeyT k = key_of(i);
            if ((k & mask) == prefix) atomicAdd(&rs->hist[(uint32_t)(k >> shift) & 255u], 1u);
        }
        __syncthreads();
        if (tid < 64) {
            uint32_t h0 = rs->hist[4 * lane], h1 = rs->hist[4 * lane + 1];
            uint32_t h2 = rs->hist[4 * lane + 2], h3 = rs->hist[4 * lane + 3];
            uint32_t own = h0 + h1 + h2 + h3;
            uint32_t s = own;
            for (int off = 1; off < 64; off <<= 1) {
                uint32_t t = __shfl_up(s, off, 64);
                if (lane >= off) s += t;
            }
            uint32_t excl = s - own;
            if (rank >= excl && rank < s) {
                uint32_t r = rank - excl;
                uint32_t b = 0;
                if (r < h0) {
                    b = 0;
                } else if (r < h0 + h1) {
                    b = 1;
                    r -= h0;
                } else if (r < h0 + h1 + h2) {
                    b = 2;
                    r -= h0 + h1;
                } else {
                    b = 3;
                    r -= h0 + h1 + h2;
                }
                rs->bin = 4 * lane + b;
                rs->rem = r;
            }
        }
        __syncthreads();
        prefix |= (KeyT)rs->bin << shift;
        mask |= (KeyT)255u << shift;
        rank = rs->rem;
    }
    __syncthreads();
    return prefix;
}

// Wave-aggregated append: lanes with `take` reserve consecutive slots of an
// LDS counter with one atomic per wave.  Returns the lane's slot (or -1).
__device__ __forceinline__ int wave_append_slot(bool take, uint32_t* counter) {
    uint64_t m = __ballot(take);
    if (m == 0) return -1;
    uint32_t lo = (uint32_t)m, hi = (uint32_t)(m >> 32);
    uint32_t below = __builtin_amdgcn_mbcnt_hi(hi, __builtin_amdgcn_mbcnt_lo(lo, 0u));
    int leader = __ffsll((unsigned long long)m) - 1;
    uint32_t base = 0;
    if ((int)(threadIdx.x & 63) == leader) base = atomicAdd(counter, (uint32_t)__popcll(m));
    base = __shfl(base, leader, 64);
    return take ? (int)(base + below) : -1;
}

// As wave_append_slot, and *after receives the counter value just after this
// wave's reservation (the same in every lane; unchanged when no lane takes).
__device__ __forceinline__ int wave_append_slot_count(bool take, uint32_t* counter,
                                                      uint32_t* after) {
    uint64_t m = __ballot(take);
    if (m == 0) {
        *after = 0;
        return -1;
    }
    uint32_t lo = (uint32_t)m, hi = (uint32_t)(m >> 32);
    uint32_t below = __builtin_amdgcn_mbcnt_hi(hi, __builtin_amdgcn_mbcnt_lo(lo, 0u));
    int leader = __ffsll((unsigned long long)m) - 1;
    uint32_t cnt = (uint32_t)__popcll(m);
    uint32_t base = 0;
    if ((int)(threadIdx.x & 63) == leader) base = atomicAdd(counter, cnt);
    base = __shfl(base, leader, 64);
    *after = base + cnt;
    return take ? (int)(base + below) : -1;
}

// v of lane (lane ^ stride), stride a power of two below 64 (a constant after
// unrolling).  Strides 1, 2 and 8 are one DPP move (quad_perm [1,0,3,2],
// quad_perm [2,3,0,1], row_ror:8), 4 is two DPP row shifts and a select, 16
// a ds_swizzle in bit mode (and 0x1f, xor 16), 32 a ds_bpermute.
__device__ __forceinline__ uint32_t shfl_xor_u32(uint32_t v, int stride) {
    const int x = (int)v;
    switch (stride) {
        case 1: return (uint32_t)__builtin_amdgcn_update_dpp(x, x, 0xB1, 0xF, 0xF, false);
        case 2: return (uint32_t)__builtin_amdgcn_update_dpp(x, x, 0x4E, 0xF, 0xF, false);
        case 4: {
            const int up = __builtin_amdgcn_update_dpp(x, x, 0x104, 0xF, 0xF, false);  // row_shl:4
            const int dn = __builtin_amdgcn_update_dpp(x, x, 0x114, 0xF, 0xF, false);  // row_shr:4
            return (uint32_t)((threadIdx.x & 4) ? dn : up);
        }
        case 8: return (uint32_t)__builtin_amdgcn_update_dpp(x, x, 0x128, 0xF, 0xF, false);
        case 16: return (uint32_t)__builtin_amdgcn_ds_swizzle(x, 0x401F);
        default: return (uint32_t)__shfl_xor(x, stride, 64);
    }
}

__device__ __forceinline__ uint64_t shfl_xor_u64(uint64_t v, int stride) {
    const uint32_t lo = shfl_xor_u32((uint32_t)v, stride);
    const uint32_t hi = shfl_xor_u32((uint32_t)(v >> 32), stride);
    return ((uint64_t)hi << 32) | lo;
}

// R separate ascending sorts of 64 32-bit keys, one per lane in k[r], their
// networks interleaved.
template <int R>
__device__ __forceinline__ void wave_sort_u32_sep(uint32_t (&k)[R]) {
    const int lane = threadIdx.x & 63;
#pragma unroll
    for (int size = 2; size <= 64; size <<= 1) {
#pragma unroll
        for (int stride = size >> 1; stride > 0; stride >>= 1) {
            const bool asc = (lane & size) == 0;
            const bool lower = (lane & stride) == 0;
#pragma unroll
            for (int r = 0; r < R; r++) {
                const uint32_t o = shfl_xor_u32(k[r], stride);
                k[r] = lower == asc ? min(o, k[r]) : max(o, k[r]);
            }
        }
    }
}

// wave_sort_regs for 32-bit keys.
template <int E>
__device__ __forceinline__ void wave_sort_u32(uint32_t (&k)[E]) {
    const int lane = threadIdx.x & 63;
#pragma unroll
    for (int size = 2; size <= 64 * E; size <<= 1) {
#pragma unroll
        for (int stride = size >> 1; stride > 0; stride >>= 1) {
            if (stride >= 64) {
                const int es = stride >> 6;
#pragma unroll
                for (int e = 0; e < E; e++) {
                    const int f = e ^ es;
                    if (f > e) {
                        const bool asc = (((e << 6) | lane) & size) == 0;
                        const uint32_t a = k[e], b = k[f];
                        k[e] = asc ? min(a, b) : max(a, b);
                        k[f] = asc ? max(a, b) : min(a, b);
                    }
                }
            } else {
#pragma unroll
                for (int e = 0; e < E; e++) {
                    const uint32_t o = shfl_xor_u32(k[e], stride);
                    const bool asc = (((e << 6) | lane) & size) == 0;
                    const bool lower = (lane & stride) == 0;
                    k[e] = lower == asc ? min(o, k[e]) : max(o, k[e]);
                }
            }
        }
    }
}

// Ascending bitonic sort of 64*E keys held by one wave, E per lane; element
// e*64 + lane lives in k[e] of that lane.  No LDS, no barriers.
template <int E>
__device__ __forceinline__ void wave_sort_regs(uint64_t (&k)[E]) {
    const int lane = threadIdx.x & 63;
#pragma unroll
    for (int size = 2; size <= 64 * E; size <<= 1) {
#pragma unroll
        for (int stride = size >> 1; stride > 0; stride >>= 1) {
            if (stride >= 64) {
                const int es = stride >> 6;
#pragma unroll
                for (int e = 0; e < E; e++) {
                    const int f = e ^ es;
                    if (f > e) {
                        const bool asc = (((e << 6) | lane) & size) == 0;
                        const uint64_t a = k[e], b = k[f];
                        const bool sw = (a > b) == asc;
                        k[e] = sw ? b : a;
                        k[f] = sw ? a : b;
                    }
                }
            } else {
#pragma unroll
                for (int e = 0; e < E; e++) {
                    const uint64_t o = shfl_xor_u64(k[e], stride);
                    const bool asc = (((e << 6) | lane) & size) == 0;
                    const bool lower = (lane & stride) == 0;
                    const bool take_min = lower == asc;
                    k[e] = take_min ? (o < k[e] ? o : k[e]) : (o > k[e] ? o : k[e]);
                }
            }
        }
    }
}
