// FAST-mode ADC scan for byte codes (codebook_size != 16): one workgroup of
// 256 threads per query, the per-query table resident in LDS, the probed
// lists streamed from HBM with two rounds of software prefetch.
//
// Reference: search_approx_internal_observed src/ivf_pq/search.rs:1175-1391
// (per probed list: residual r = q - c, compute_adc_table_into
// src/ivf_pq/pq.rs:232-251, adc_batch_256_into src/pq_simd.rs:330-369);
// finish_top_k_by_distance search.rs:64-75.
//
// Ranking.  The reference distance of an entry x in list l is
//     ||r - x_r||^2 = ||q - c||^2 + (||x_r||^2 + 2 c.x_r) - 2 q.x_r .
// The middle term b(x) is stored per list position at upload, the first is
// one value per probed list, the last is a per-query table T2[m][k] =
// -2 q_m.cw_mk, so the scan needs one table per query (not one per probed
// list) and one 4-byte load per entry besides its codes.  Every approximate
// distance a is within tau of the reference's float32 distance e
// (fast_tau, below).
//
// Selection.  Entries with fkey(a) <= thr are appended to an LDS buffer;
// when the buffer fills, a block radix select finds the keep-th smallest key
// T and the buffer is compacted to the entries <= T, which become the new
// threshold.  The buffer therefore always holds every scanned entry with
// key <= thr.  At the end, with A_k the k-th smallest approximate distance,
// the reference's top-k lies inside R = {a <= A_k + 2 tau}: the k entries with
// the smallest a have e <= A_k + tau, so the k-th smallest e is at most
// A_k + tau, and any entry of the exact top-k has a <= e + tau <= A_k + 2 tau.
// If the buffer provably holds R (A_k + 2 tau <= thr), R is rescored with the
// reference's arithmetic and sorted by (distance, insertion index);
// otherwise the query is flagged and rerun by the EXACT kernel.
#include <hip/hip_ext.h>

#include "vgpu_device.h"
#include "vgpu_launch.h"

namespace vgpu {

#define FS_U 1                          // entries per thread per round
#define FS_ROUND (VGPU_BLOCK * FS_U)    // entries per round

// Codes of one list entry held in registers.
template <int MT>
struct CodeRow {
    uint32_t w[MT >= 4 ? MT / 4 : 1];
};

template <int MT>
__device__ __forceinline__ void load_row(CodeRow<MT>& r, const uint8_t* __restrict__ p) {
    if constexpr (MT % 16 == 0) {
        const uint4* v = reinterpret_cast<const uint4*>(p);
#pragma unroll
        for (int i = 0; i < MT / 16; i++) {
            uint4 x = v[i];
            r.w[4 * i] = x.x;
            r.w[4 * i + 1] = x.y;
            r.w[4 * i + 2] = x.z;
            r.w[4 * i + 3] = x.w;
        }
    } else if constexpr (MT == 8) {
        uint2 x = *reinterpret_cast<const uint2*>(p);
        r.w[0] = x.x;
        r.w[1] = x.y;
    } else {
        static_assert(MT == 4, "row width");
        r.w[0] = *reinterpret_cast<const uint32_t*>(p);
    }
}

// sum_m lut[m*K + code_m] with four partial sums (ranking only; the order of
// the additions is covered by tau).  The table is a static LDS array at a
// fixed address, so each lookup is one byte-select shift plus an
// immediate-offset LDS read.
template <int MT, int KT>
__device__ __forceinline__ float row_sum(const CodeRow<MT>& r, const float* __restrict__ lut) {
    static_assert(MT >= 4 && MT % 4 == 0, "row width");
    const uint32_t w0 = r.w[0];
    float s0 = lut[0 * KT + (w0 & 0xffu)];
    float s1 = lut[1 * KT + ((w0 >> 8) & 0xffu)];
    float s2 = lut[2 * KT + ((w0 >> 16) & 0xffu)];
    float s3 = lut[3 * KT + (w0 >> 24)];
#pragma unroll
    for (int i = 1; i < MT / 4; i++) {
        const uint32_t w = r.w[i];
        s0 += lut[(4 * i + 0) * KT + (w & 0xffu)];
        s1 += lut[(4 * i + 1) * KT + ((w >> 8) & 0xffu)];
        s2 += lut[(4 * i + 2) * KT + ((w >> 16) & 0xffu)];
        s3 += lut[(4 * i + 3) * KT + (w >> 24)];
    }
    return (s0 + s1) + (s2 + s3);
}

// Generic M / K: bytes straight from global memory.
__device__ __forceinline__ float row_sum_generic(const uint8_t* __restrict__ p,
                                                 const float* __restrict__ lut, int M, int K) {
    float s0 = 0.0f, s1 = 0.0f;
    int m = 0;
    for (; m + 1 < M; m += 2) {
        s0 += lut[m * K + p[m]];
        s1 += lut[(m + 1) * K + p[m + 1]];
    }
    if (m < M) s0 += lut[m * K + p[m]];
    return s0 + s1;
}

// Bound on |a - e| for ||q|| <= qn, ||c|| <= cmax, ||x_r|| <= rmax and
// ||q - c||^2 <= t0max (u = 2^-24).  With rr = sqrt(t0max) + rmax >= ||r - x_r||:
//   |e - D| <= (ds + M) u rr^2 + 2u (||q - c|| rr + rr^2)     (reference arithmetic)
//   |a - D| <= (d + M + ds + 4) u (t0max + rmax^2 + 2 (cmax + qn) rmax)
// where D is the real-number distance; both are below
// (d + M + ds + 8) u S with S = 2 (qn + cmax) rmax + 2 rmax^2 + 2 rr^2, which
// is taken with a factor of 4 to spare.
__device__ __forceinline__ float fast_tau(int d, int M, int ds, float qn, float cmax, float rmax,
                                          float t0max) {
    const float u = 5.9604645e-08f;
    float rr = sqrtf(t0max) + rmax;
    float S = 2.0f * (qn + cmax) * rmax + 2.0f * rmax * rmax + 2.0f * rr * rr;
    return 4.0f * (float)(d + M + ds + 8) * u * S + 1e-30f;
}

struct FastLds {
    float* lut;      // [M * max(K, 64)] table, then rescoring scratch
    uint64_t* keys;  // [buf] (fkey(a) << 32) | position
    float* qs;       // [d]
    uint32_t* lid;   // [P]
    uint32_t* lbeg;  // [P]
    uint32_t* llen;  // [P]
    uint32_t* pref;  // [P + 1]
    float* term0;    // [P] ||q - c||^2
    uint2* bt;       // [P] (lbeg - pref as u32, bits of term0): one read per entry
    RadixScratch* rs;
    uint32_t* misc;  // [0] count [1] thr [2] lost ties [3..4] flush flags by round parity
                     // [5] entries evicted by flushes [6] flushes
};

__host__ __device__ inline size_t fs8_align(size_t x) { return (x + 15) & ~(size_t)15; }

__host__ __device__ inline int fs8_buf(int keep) {
    int need = keep + FS_ROUND;
    int b = 1;
    while (b < need) b <<= 1;
    return b;
}

// Dynamic LDS layout; the table region is omitted when the kernel holds the
// table in a static array (static_lut: compile-time M and K = 256).
__host__ __device__ inline size_t fs8_layout(int d, int M, int K, int P, int buf, bool static_lut,
                                             size_t* off) {
    size_t o = 0;
    const int KL = K > 64 ? K : 64;
    off[0] = o; o = static_lut ? 0 : fs8_align(o + (size_t)M * KL * 4);  // lut
    off[1] = o; o = fs8_align(o + (size_t)buf * 8);        // keys
    off[2] = o; o = fs8_align(o + (size_t)d * 4);          // qs
    off[3] = o; o = fs8_align(o + (size_t)P * 4);          // lid
    off[4] = o; o = fs8_align(o + (size_t)P * 4);          // lbeg
    off[5] = o; o = fs8_align(o + (size_t)P * 4);          // llen
    off[6] = o; o = fs8_align(o + (size_t)(P + 1) * 4);    // pref
    off[7] = o; o = fs8_align(o + (size_t)P * 4);          // term0
    off[8] = o; o = fs8_align(o + sizeof(RadixScratch));   // radix scratch
    off[9] = o; o = fs8_align(o + 8 * 4);                  // misc
    off[10] = o; o = fs8_align(o + (size_t)P * 8);         // bt
    return o;
}

__device__ inline FastLds fs8_carve(char* smem, float* static_lut, int d, int M, int K, int P,
                                    int buf) {
    size_t off[11];
    fs8_layout(d, M, K, P, buf, static_lut != nullptr, off);
    FastLds s;
    s.lut = static_lut ? static_lut : (float*)(smem + off[0]);
    s.keys = (uint64_t*)(smem + off[1]);
    s.qs = (float*)(smem + off[2]);
    s.lid = (uint32_t*)(smem + off[3]);
    s.lbeg = (uint32_t*)(smem + off[4]);
    s.llen = (uint32_t*)(smem + off[5]);
    s.pref = (uint32_t*)(smem + off[6]);
    s.term0 = (float*)(smem + off[7]);
    s.rs = (RadixScratch*)(smem + off[8]);
    s.misc = (uint32_t*)(smem + off[9]);
    s.bt = (uint2*)(smem + off[10]);
    return s;
}

// Keep the buffer entries whose high word is <= T (in place, chunk by chunk:
// a chunk is read into registers before any of its slots are rewritten, and
// the compacted prefix never passes the end of the chunk being read).  Keys
// carry t, the entry's index in the concatenated probed lists; with
// `relabel`, each kept key is rewritten as (probe slot << 32) | position, the
// slot found by binary search over the list prefix sums.
__device__ inline uint32_t fs8_compact(FastLds& s, uint32_t n, uint32_t T, bool relabel, int P) {
    const int tid = threadIdx.x;
    __syncthreads();
    if (tid == 0) s.misc[0] = 0;
    __syncthreads();
    for (uint32_t c0 = 0; c0 < n; c0 += VGPU_BLOCK) {
        const uint32_t i = c0 + tid;
        uint64_t v = i < n ? s.keys[i] : ~0ull;
        bool take = i < n && (uint32_t)(v >> 32) <= T;
        __syncthreads();
        if (take && relabel) {
            // the largest slot p < P with pref[p] <= t is the non-empty list holding t
            const uint32_t t = (uint32_t)v;
            uint32_t lo = 0, hi = (uint32_t)P;
            while (hi - lo > 1u) {
                const uint32_t mid = (lo + hi) >> 1;
                if (s.pref[mid] <= t) lo = mid;
                else hi = mid;
            }
            v = ((uint64_t)lo << 32) | (s.lbeg[lo] + (t - s.pref[lo]));
        }
        int slot = wave_append_slot(take, &s.misc[0]);
        if (take) s.keys[slot] = v;
        __syncthreads();
    }
    return s.misc[0];
}

// An upper bound U on the rank-th smallest (0-based) high word of the buffer
// keys (n > rank), from one 256-bin histogram over the 8 bits below the
// common prefix of the smallest and largest high word: U is the top of the
// bin holding rank, so every key <= the rank-th is <= U and the keys <= U are
// those of the bins up to it.  When those number more than `limit`, the exact
// radix select is taken instead.  All threads call it.
__device__ uint32_t fs8_select_upper(FastLds& s, uint32_t n, uint32_t rank, uint32_t limit) {
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    uint32_t mn = 0xffffffffu, mx = 0u;
    for (uint32_t i = tid; i < n; i += VGPU_BLOCK) {
        const uint32_t h = (uint32_t)(s.keys[i] >> 32);
        mn = h < mn ? h : mn;
        mx = h > mx ? h : mx;
    }
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const uint32_t a = shfl_xor_u32(mn, o), b = shfl_xor_u32(mx, o);
        mn = a < mn ? a : mn;
        mx = b > mx ? b : mx;
    }
    __syncthreads();  // the scratch may still be read by a previous select
    if (lane == 0) {
        s.rs->hist[wave] = mn;
        s.rs->hist[8 + wave] = mx;
    }
    __syncthreads();
#pragma unroll
    for (int w = 0; w < VGPU_BLOCK / 64; w++) {
        const uint32_t a = s.rs->hist[w], b = s.rs->hist[8 + w];
        mn = a < mn ? a : mn;
        mx = b > mx ? b : mx;
    }
    if (mn == mx) return mx;
    const int sbit = 31 - __clz(mn ^ mx);  // highest differing bit
    const int shift = sbit > 7 ? sbit - 7 : 0;
    __syncthreads();
    for (int i = tid; i < 256; i += VGPU_BLOCK) s.rs->hist[i] = 0u;
    __syncthreads();
    for (uint32_t i = tid; i < n; i += VGPU_BLOCK)
        atomicAdd(&s.rs->hist[((uint32_t)(s.keys[i] >> 32) >> shift) & 255u], 1u);
    __syncthreads();
    if (tid < 64) {
        const uint32_t h0 = s.rs->hist[4 * lane], h1 = s.rs->hist[4 * lane + 1];
        const uint32_t h2 = s.rs->hist[4 * lane + 2], h3 = s.rs->hist[4 * lane + 3];
        const uint32_t own = h0 + h1 + h2 + h3;
        uint32_t incl = own;
#pragma unroll
        for (int o = 1; o < 64; o <<= 1) {
            const uint32_t x = __shfl_up(incl, o, 64);
            if (lane >= o) incl += x;
        }
        const uint32_t excl = incl - own;
        if (rank >= excl && rank < incl) {
            uint32_t b = 3, upto = incl;  // keys in bins <= b
            if (rank < excl + h0) { b = 0; upto = excl + h0; }
            else if (rank < excl + h0 + h1) { b = 1; upto = excl + h0 + h1; }
            else if (rank < excl + h0 + h1 + h2) { b = 2; upto = excl + h0 + h1 + h2; }
            s.rs->bin = 4 * lane + b;
            s.rs->rem = upto;
        }
    }
    __syncthreads();
    const uint32_t b = s.rs->bin, upto = s.rs->rem;
    if (upto > limit) {  // a heavy bin: exact select
        auto hk = [&](int i) -> uint32_t { return (uint32_t)(s.keys[i] >> 32); };
        return block_radix_select<uint32_t>(hk, (int)n, rank, s.rs);
    }
    const uint32_t low = (1u << shift) - 1u;
    const uint32_t base = sbit >= 31 ? 0u : (mn & ~((2u << sbit) - 1u));  // common prefix
    return base | (b << shift) | low;
}

// Buffer full: keep the `keep` smallest keys (plus the rest of their
// histogram bin); at most `cap` survive, otherwise the query is marked failed.
// Clears the flag of `parity`.
__device__ inline void fs8_flush(FastLds& s, int keep, uint32_t cap, int parity) {
    __syncthreads();
    const uint32_t n = s.misc[0];
    if (threadIdx.x == 0) s.misc[3 + parity] = 0u;
    if (n <= (uint32_t)keep) {
        __syncthreads();
        return;
    }
    const uint32_t T = fs8_select_upper(s, n, (uint32_t)(keep - 1), cap);
    const uint32_t kept = fs8_compact(s, n, T, false, 0);
    __syncthreads();
    if (threadIdx.x == 0) {
        if (kept > cap) {
            s.misc[0] = cap;
            s.misc[2] = 1u;
        }
        s.misc[1] = T;
        s.misc[5] += n - (kept < cap ? kept : cap);  // entries evicted
        s.misc[6] += 1u;
    }
    __syncthreads();
}

// Per-thread state of the entries one thread handles in one round.  The
// loads are unconditional (a slot past the end reads position 0, which exists
// whenever anything is scanned) so the compiler can wait for one round's
// loads while the next rounds' are still in flight.
template <int MT>
struct RoundRegs {
    CodeRow<MT> row[FS_U];
    float bias[FS_U];
    float t0[FS_U];    // ||q - c||^2 of the entry's list
    uint32_t pos[FS_U];// position (code row), generic path only
    uint32_t t[FS_U];  // index in the concatenated probed lists; 0xffffffff = no entry
};

// Entry t = rbase + u * VGPU_BLOCK + tid.  Each wave's 64 entries of a slot
// are consecutive, so the wave keeps one uniform cursor `cw` (the probed list
// holding the start of its next window; windows only move forward) and a lane
// finds its list by counting the list starts inside the window (usually none
// or one).  Empty lists repeat a start and are counted over.
template <int MT>
__device__ __forceinline__ void fs8_fetch(const DevIndex& ix, const FastLds& s, uint32_t rbase,
                                          uint32_t total, int P, int& cw, RoundRegs<MT>& g) {
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
#pragma unroll
    for (int u = 0; u < FS_U; u++) {
        const uint32_t wb = rbase + (uint32_t)u * VGPU_BLOCK + wave * 64u;  // window start
        const uint32_t t = wb + lane;
        const bool valid = t < total;
        while (cw + 1 < P && __builtin_amdgcn_readfirstlane(s.pref[cw + 1]) <= wb) cw++;
        int lst = cw;
        for (int j = cw + 1; j < P; j++) {
            const uint32_t b = __builtin_amdgcn_readfirstlane(s.pref[j]);
            if (b >= wb + 64u) break;
            lst += t >= b ? 1 : 0;
        }
        const uint2 e = s.bt[lst];
        const uint32_t pos = valid ? e.x + t : 0u;
        g.pos[u] = pos;
        g.t[u] = valid ? t : 0xffffffffu;
        g.t0[u] = __uint_as_float(e.y);
        if constexpr (MT > 0) load_row<MT>(g.row[u], ix.codes + (size_t)pos * MT);
        g.bias[u] = ix.bias[pos];
    }
}

// Score one round of entries and append those with fkey(a) <= thr, with one
// LDS atomic per wave.  A wave whose appends took the buffer past `cap`
// raises flag misc[3 + parity]: the final count is the largest count any wave
// saw, so the flag is raised exactly when the buffer needs a flush.  The two
// parities alternate between rounds, and a raised flag is cleared inside the
// flush, so a flag is never written while another wave may still read it.
// Every thread of the block calls this (all lanes active).  The second pass
// (RETRY) appends only keys in (lo, thr]: the buffer already holds every key
// <= lo.
template <int MT, int KT, bool RETRY>
__device__ __forceinline__ void fs8_consume(const DevIndex& ix, FastLds& s, const float* lut_static,
                                            const RoundRegs<MT>& g, uint32_t thr, uint32_t lo,
                                            uint32_t cap, int parity) {
    const int lane = threadIdx.x & 63;
    bool take[FS_U];
    uint32_t fk[FS_U], before[FS_U];
    uint64_t mask[FS_U];
    uint32_t tot = 0;
#pragma unroll
    for (int u = 0; u < FS_U; u++) {
        const bool ok = g.t[u] != 0xffffffffu;
        float dist;
        if constexpr (MT > 0 && KT > 0) {
            dist = (g.t0[u] + g.bias[u]) + row_sum<MT, KT>(g.row[u], lut_static);
        } else {
            dist = (g.t0[u] + g.bias[u]) +
                   row_sum_generic(ix.codes + (size_t)g.pos[u] * ix.M, s.lut, ix.M, ix.K);
        }
        fk[u] = fkey(dist);
        take[u] = ok && fk[u] <= thr && (!RETRY || fk[u] > lo);
        mask[u] = __ballot(take[u]);
        before[u] = tot;
        tot += (uint32_t)__popcll(mask[u]);
    }
    if (tot == 0) return;  // wave-uniform
    uint32_t base = 0;
    if (lane == 0) base = atomicAdd(&s.misc[0], tot);
    base = __builtin_amdgcn_readfirstlane(base);
#pragma unroll
    for (int u = 0; u < FS_U; u++) {
        if (take[u]) {
            const uint32_t below = __builtin_amdgcn_mbcnt_hi(
                (uint32_t)(mask[u] >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)mask[u], 0u));
            s.keys[base + before[u] + below] = ((uint64_t)fk[u] << 32) | g.t[u];
        }
    }
    if (base + tot > cap && lane == 0) s.misc[3 + parity] = 1u;
}

// DS consecutive floats into registers (vector loads when aligned).
template <int DS>
__device__ __forceinline__ void load_vec(const float* __restrict__ p, float* v) {
    if constexpr (DS % 4 == 0) {
#pragma unroll
        for (int i = 0; i < DS / 4; i++) {
            const float4 x = reinterpret_cast<const float4*>(p)[i];
            v[4 * i] = x.x;
            v[4 * i + 1] = x.y;
            v[4 * i + 2] = x.z;
            v[4 * i + 3] = x.w;
        }
    } else if constexpr (DS == 2) {
        const float2 x = reinterpret_cast<const float2*>(p)[0];
        v[0] = x.x;
        v[1] = x.y;
    } else {
#pragma unroll
        for (int j = 0; j < DS; j++) v[j] = p[j];
    }
}

// The reference's distance contribution of codebook m for one entry
// (pq.rs:232-251 on r = q - c, search.rs:1242-1245): sub, sub, mul, add in
// dimension order, no contraction.
template <int DS>
__device__ __forceinline__ float exact_sub_distance(const float* qm, const float* c,
                                                    const float* cw, int ds) {
    float e = 0.0f;
    if constexpr (DS > 0) {
        float cv[DS], wv[DS];
        load_vec<DS>(c, cv);
        load_vec<DS>(cw, wv);
#pragma unroll
        for (int j = 0; j < DS; j++) {
            const float r = __fsub_rn(qm[j], cv[j]);
            const float diff = __fsub_rn(r, wv[j]);
            e = __fadd_rn(e, __fmul_rn(diff, diff));
        }
    } else {
        for (int j = 0; j < ds; j++) {
            const float r = __fsub_rn(qm[j], c[j]);
            const float diff = __fsub_rn(r, cw[j]);
            e = __fadd_rn(e, __fmul_rn(diff, diff));
        }
    }
    return e;
}

// MT, KT, DS: compile-time codebooks, codebook size and subvector dimension
// (0 = read from the index at run time).
template <int MT, int KT, int DS>
__global__ __launch_bounds__(256) void scan8_fast_kernel(DevIndex ix, ScanArgs a, int buf) {
    constexpr bool kStatic = MT > 0 && KT >= 64;
    constexpr int D = MT * DS;  // compile-time dimension when > 0
    __shared__ __align__(16) float slut[kStatic ? MT * KT : 1];
    extern __shared__ __align__(16) char smem[];
    const int q = blockIdx.x;
    if (q >= a.nq) return;
    const int tid = threadIdx.x, lane = tid & 63;
    const int d = D > 0 ? D : ix.d, M = MT > 0 ? MT : ix.M, K = KT > 0 ? KT : ix.K;
    const int ds = DS > 0 ? DS : ix.ds, P = a.P;
    FastLds s = fs8_carve(smem, kStatic ? slut : nullptr, d, M, K, P, buf);

    // ---- prologue: query, probed lists, ||q - c||^2, the per-query table.
    for (int j = tid; j < d; j += VGPU_BLOCK) s.qs[j] = a.qn[(size_t)q * d + j];
    for (int p = tid; p < P; p += VGPU_BLOCK) {
        const uint32_t l = a.probe[(size_t)q * P + p];
        const bool ok = l < (uint32_t)ix.L;  // no such list: scanned as empty
        const uint32_t b = ok ? ix.offsets[l] : 0u;
        s.lid[p] = ok ? l : 0u;
        s.lbeg[p] = b;
        s.llen[p] = ok ? ix.offsets[l + 1] - b : 0u;
    }
    if (tid < 8) s.misc[tid] = tid == 1 ? 0xffffffffu : 0u;  // count 0, thr +inf, flags 0
    __syncthreads();
    if (tid < 64) {  // exclusive prefix of the list lengths
        uint32_t carry = 0;
        for (int p0 = 0; p0 < P; p0 += 64) {
            const int p = p0 + lane;
            const uint32_t own = p < P ? s.llen[p] : 0u;
            uint32_t x = own;
            for (int o = 1; o < 64; o <<= 1) {
                uint32_t y = __shfl_up(x, o, 64);
                if (lane >= o) x += y;
            }
            if (p < P) s.pref[p] = carry + x - own;
            carry += __shfl(x, 63, 64);
        }
        if (lane == 0) s.pref[P] = carry;
    }
    {  // ||q - c||^2: eight lanes per probed list (ranking only: any order)
        const int g = tid >> 3, sub = tid & 7;
        for (int p0 = 0; p0 < P; p0 += VGPU_BLOCK / 8) {
            const int p = p0 + g;
            float acc = 0.0f;
            if (p < P) {
                const float* c = ix.centroids + (size_t)s.lid[p] * d;
                if constexpr (D > 0 && D % 32 == 0) {
                    float cv[D / 8];
#pragma unroll
                    for (int i = 0; i < D / 32; i++) load_vec<4>(c + 32 * i + 4 * sub, cv + 4 * i);
#pragma unroll
                    for (int i = 0; i < D / 32; i++)
#pragma unroll
                        for (int j = 0; j < 4; j++) {
                            const float t = s.qs[32 * i + 4 * sub + j] - cv[4 * i + j];
                            acc = __builtin_fmaf(t, t, acc);
                        }
                } else {
                    for (int j = sub; j < d; j += 8) {
                        const float t = s.qs[j] - c[j];
                        acc = __builtin_fmaf(t, t, acc);
                    }
                }
            }
            acc += __uint_as_float(shfl_xor_u32(__float_as_uint(acc), 1));
            acc += __uint_as_float(shfl_xor_u32(__float_as_uint(acc), 2));
            acc += __uint_as_float(shfl_xor_u32(__float_as_uint(acc), 4));
            if (p < P && sub == 0) s.term0[p] = acc;
        }
    }
    // T2[m][k] = -2 q_m . cw_mk (ranking only: FMA allowed)
    if constexpr (MT > 0 && KT > 0 && DS > 0 && (MT * KT) % VGPU_BLOCK == 0) {
        constexpr int NE = MT * KT / VGPU_BLOCK;           // entries per thread
        constexpr int G = DS >= 8 ? 4 : (NE < 8 ? NE : 8);  // entries whose loads fly together
        static_assert(NE % G == 0, "table split");
#pragma unroll
        for (int g0 = 0; g0 < NE; g0 += G) {
            float wv[G][DS];
#pragma unroll
            for (int i = 0; i < G; i++)
                load_vec<DS>(ix.codebooks + (size_t)((g0 + i) * VGPU_BLOCK + tid) * DS, wv[i]);
#pragma unroll
            for (int i = 0; i < G; i++) {
                const int e = (g0 + i) * VGPU_BLOCK + tid;
                const float* qm = s.qs + (e / KT) * DS;
                float acc = 0.0f;
#pragma unroll
                for (int j = 0; j < DS; j++) acc = __builtin_fmaf(qm[j], wv[i][j], acc);
                s.lut[e] = -2.0f * acc;
            }
        }
    } else {
        for (int e = tid; e < M * K; e += VGPU_BLOCK) {
            const float* cw = ix.codebooks + (size_t)e * ds;
            const float* qm = s.qs + (e / K) * ds;
            float acc = 0.0f;
            for (int j = 0; j < ds; j++) acc = __builtin_fmaf(qm[j], cw[j], acc);
            s.lut[e] = -2.0f * acc;
        }
    }
    for (int p = tid; p < P; p += VGPU_BLOCK)
        s.bt[p] = make_uint2(s.lbeg[p] - s.pref[p], __float_as_uint(s.term0[p]));
    __syncthreads();

    // ---- scan: FS_ROUND entries per round, the next two rounds' loads in
    // flight (a ring of three register sets).  Round r uses flag parity r & 1.
    const uint32_t total = s.pref[P];
    const int keep = a.kk;
    const uint32_t cap = (uint32_t)(buf - FS_ROUND);
    int cur = 0;
    RoundRegs<MT> ga, gb, gc;
    if (total > 0) {
        fs8_fetch<MT>(ix, s, 0, total, P, cur, ga);
        fs8_fetch<MT>(ix, s, FS_ROUND, total, P, cur, gb);
    }
#define FS8_STEP(CONSUME, NEXT, R)                                                     \
    {                                                                                  \
        const uint32_t rbase = (R) * FS_ROUND;                                         \
        const int par = (int)((R) & 1u);                                               \
        fs8_fetch<MT>(ix, s, rbase + 2 * FS_ROUND, total, P, cur, NEXT);                  \
        fs8_consume<MT, KT, false>(ix, s, slut, CONSUME, s.misc[1], 0u, cap, par);     \
        __syncthreads();                                                               \
        if (s.misc[3 + par]) fs8_flush(s, keep, cap, par);                             \
        if (rbase + FS_ROUND >= total) break;                                          \
    }
    for (uint32_t r = 0; r * FS_ROUND < total; r += 3) {
        FS8_STEP(ga, gc, r)
        FS8_STEP(gb, ga, r + 1)
        FS8_STEP(gc, gb, r + 2)
    }
#undef FS8_STEP
    __syncthreads();

    // ---- proof that the buffer holds R, then rescoring.
    uint32_t n = s.misc[0];
    const uint32_t thr = s.misc[1];
    const int kout = a.kout;
    bool fail = s.misc[2] != 0u;
    bool retried = false;
    uint32_t bk = 0xffffffffu;
    if (!fail && n > (uint32_t)kout) {
        // an upper bound on A_k: R grows by at most the rest of A_k's bin
        const uint32_t Ak = fs8_select_upper(s, n, (uint32_t)(kout - 1), 0xffffffffu);
        float t0max = 0.0f;
        for (int p = 0; p < P; p++) t0max = fmaxf(t0max, s.term0[p]);
        const float tau = fast_tau(d, M, ds, a.qnorm[q], ix.cmax, ix.rmax, t0max);
        const float bound = fkey_to_float(Ak) + 2.0f * tau;
        bk = fkey(bound);
        bk = bk < 0xfffffffeu ? bk + 1u : 0xffffffffu;  // one ulp to spare
        if (thr != 0xffffffffu && bk > thr) {
            // Second pass: the buffer holds every key <= thr; add the keys in
            // (thr, bk] with no flush, so afterwards it holds all of R.  More
            // than the buffer holds fails the query (EXACT rerun).
            retried = true;
            if (tid == 0) {
                s.misc[1] = bk;
                s.misc[3] = s.misc[4] = 0u;
            }
            __syncthreads();
            cur = 0;
            fs8_fetch<MT>(ix, s, 0, total, P, cur, ga);
            for (uint32_t rb = 0; rb < total; rb += 2 * FS_ROUND) {
                fs8_fetch<MT>(ix, s, rb + FS_ROUND, total, P, cur, gb);
                fs8_consume<MT, KT, true>(ix, s, slut, ga, bk, thr, cap, 0);
                __syncthreads();
                if (s.misc[3]) break;
                if (rb + FS_ROUND >= total) break;
                fs8_fetch<MT>(ix, s, rb + 2 * FS_ROUND, total, P, cur, ga);
                fs8_consume<MT, KT, true>(ix, s, slut, gb, bk, thr, cap, 1);
                __syncthreads();
                if (s.misc[4]) break;
            }
            __syncthreads();
            n = s.misc[0];
            if (s.misc[3] | s.misc[4]) {
                fail = true;
                if (tid == 0) s.misc[2] = 1u;
            }
            __syncthreads();
        }
    }
    if (tid == 0) {
        uint32_t* st = a.qstat + (size_t)q * QSTAT_WORDS;
        st[0] = total;
        st[1] = s.misc[6];
        st[2] = s.misc[5] + n;  // appended = evicted + still held
        st[3] = (fail ? (1u | (s.misc[2] ? 2u : 0u)) : 0u) | (retried ? 4u : 0u);
        if (fail) a.flag_list[atomicAdd(a.flag_count, 1u)] = (uint32_t)q;
    }
    if (fail) return;
    n = fs8_compact(s, n, bk, true, P);  // R, keys relabelled (probe slot, position)

    // Two threads per entry (codebooks 0 .. M/2 - 1 and M/2 .. M - 1) when the
    // probed lists' residuals r = q - c fit the idle table region: each thread
    // loads its half code row, then its codewords in batches; r comes from LDS
    // (the same single subtraction exact_sub_distance makes).  The first
    // thread adds its sub-distances in codebook order from 0.0 and continues
    // with its partner's, handed over by a lane shuffle (pq_simd.rs:349-355).
    if constexpr (MT == 8 || MT == 16 || MT == 32) {
        if constexpr (KT > 0 && DS > 0) {
            if ((size_t)P * D <= (size_t)MT * KT && n <= (uint32_t)(VGPU_BLOCK / 2)) {
                constexpr int H = MT / 2;                 // codebooks per thread
                constexpr int CB0 = DS >= 8 ? 4 : 8;
                constexpr int CB = CB0 < H ? CB0 : H;     // codewords in flight
                static_assert(H % CB == 0 && H % 4 == 0, "codebook batches");
                constexpr int HW = H / 4;                 // code words per half row
                const uint32_t i = (uint32_t)tid >> 1, half = (uint32_t)tid & 1u;
                const bool act = i < n;
                const uint64_t v = act ? s.keys[i] : 0ull;
                const uint32_t pos = (uint32_t)v, p = (uint32_t)(v >> 32);
                uint32_t cwd[HW];
#pragma unroll
                for (int w = 0; w < HW; w++) cwd[w] = 0u;
                if (act) {
                    const uint8_t* cp = ix.codes + (size_t)pos * MT + half * H;
                    if constexpr (HW == 1) cwd[0] = *reinterpret_cast<const uint32_t*>(cp);
                    else if constexpr (HW == 2) {
                        const uint2 x = *reinterpret_cast<const uint2*>(cp);
                        cwd[0] = x.x; cwd[1] = x.y;
                    } else {
                        const uint4 x = *reinterpret_cast<const uint4*>(cp);
                        cwd[0] = x.x; cwd[1] = x.y; cwd[2] = x.z; cwd[3] = x.w;
                    }
                }
                for (int e = tid; e < P * (D / 4); e += VGPU_BLOCK) {  // residual table
                    const int pp = e / (D / 4), j = 4 * (e % (D / 4));
                    const float4 c = *reinterpret_cast<const float4*>(ix.centroids + (size_t)s.lid[pp] * D + j);
                    float* o = s.lut + pp * D + j;
                    o[0] = __fsub_rn(s.qs[j], c.x);
                    o[1] = __fsub_rn(s.qs[j + 1], c.y);
                    o[2] = __fsub_rn(s.qs[j + 2], c.z);
                    o[3] = __fsub_rn(s.qs[j + 3], c.w);
                }
                __syncthreads();
                float ev[H];
                const float* rrow = s.lut + (size_t)p * D + half * H * DS;
#pragma unroll
                for (int h0 = 0; h0 < H; h0 += CB) {
                    float wv[CB][DS];
#pragma unroll
                    for (int b = 0; b < CB; b++) {
                        const int h = h0 + b, m = (int)half * H + h;
                        const uint32_t code = (cwd[h >> 2] >> (8 * (h & 3))) & 0xffu;
                        load_vec<DS>(ix.codebooks + ((size_t)m * KT + code) * DS, wv[b]);
                    }
#pragma unroll
                    for (int b = 0; b < CB; b++) {
                        float e = 0.0f;
#pragma unroll
                        for (int j = 0; j < DS; j++) {
                            const float diff = __fsub_rn(rrow[(h0 + b) * DS + j], wv[b][j]);
                            e = __fadd_rn(e, __fmul_rn(diff, diff));
                        }
                        ev[h0 + b] = e;
                    }
                }
                float total_e = 0.0f;  // codebooks 0 .. H - 1 (first thread)
#pragma unroll
                for (int h = 0; h < H; h++) total_e = __fadd_rn(total_e, ev[h]);
#pragma unroll
                for (int h = 0; h < H; h++)  // then the partner's H .. M - 1
                    total_e = __fadd_rn(total_e, __uint_as_float(shfl_xor_u32(__float_as_uint(ev[h]), 1)));
                __syncthreads();  // every key of R read above before any is rewritten
                if (act && half == 0) s.keys[i] = cand_key(total_e, ix.list_ids[pos]);
                __syncthreads();
                goto rescored;
            }
        }
    }
    {
    // Rescoring chunks of KL entries: their code rows are staged in the table
    // region after the KL x M partial distances, so the codeword loads do not
    // wait on a dependent global load.
    const int KL = K > 64 ? K / 2 : 32;
    uint8_t* scodes = reinterpret_cast<uint8_t*>(s.lut + (size_t)KL * M);
    for (uint32_t c0 = 0; c0 < n; c0 += (uint32_t)KL) {
        const uint32_t cn = min((uint32_t)KL, n - c0);
        if constexpr (MT > 0 && MT % 16 == 0) {  // 16-byte pieces of code rows
            for (uint32_t t = tid; t < cn * (uint32_t)(MT / 16); t += VGPU_BLOCK) {
                const uint32_t i = t / (uint32_t)(MT / 16), w = t % (uint32_t)(MT / 16);
                const uint32_t pos = (uint32_t)s.keys[c0 + i];
                reinterpret_cast<uint4*>(scodes)[t] =
                    reinterpret_cast<const uint4*>(ix.codes + (size_t)pos * MT)[w];
            }
        } else {
            for (uint32_t t = tid; t < cn * (uint32_t)M; t += VGPU_BLOCK) {
                const uint32_t pos = (uint32_t)s.keys[c0 + t / (uint32_t)M];
                scodes[t] = ix.codes[(size_t)pos * M + t % (uint32_t)M];
            }
        }
        __syncthreads();
#pragma unroll 2
        for (uint32_t t = tid; t < cn * (uint32_t)M; t += VGPU_BLOCK) {
            const uint32_t i = c0 + t / (uint32_t)M;
            const int m = (int)(t % (uint32_t)M);
            const uint64_t v = s.keys[i];
            const uint32_t p = (uint32_t)(v >> 32);
            const uint8_t code = scodes[t];
            const float* cw = ix.codebooks + ((size_t)m * K + code) * ds;
            const float* c = ix.centroids + (size_t)s.lid[p] * d + m * ds;
            s.lut[t] = exact_sub_distance<DS>(s.qs + m * ds, c, cw, ds);
        }
        __syncthreads();
        for (uint32_t i = c0 + tid; i < c0 + cn; i += VGPU_BLOCK) {
            const float* em = s.lut + (size_t)(i - c0) * M;
            float total_e = 0.0f;  // pq_simd.rs:349-355: m = 0..M-1 from 0.0
            for (int m = 0; m < M; m++) total_e = __fadd_rn(total_e, em[m]);
            const uint32_t pos = (uint32_t)s.keys[i];
            s.keys[i] = cand_key(total_e, ix.list_ids[pos]);
        }
        __syncthreads();
    }
    }
rescored:
    if (n <= 256) {  // one wave sorts in registers; no block barriers below
        if (tid >= 64) return;
        auto emit = [&](int j, uint64_t key) {
            const size_t o = (size_t)q * kout + j;
            if ((uint32_t)j < n) {
                a.out_vidx[o] = (uint32_t)key;
                a.out_dist[o] = key_dist(key);
            } else {
                a.out_vidx[o] = 0xffffffffu;
                a.out_dist[o] = __int_as_float(0x7f800000);
            }
        };
        int done = 64;
        if (n <= 64) {
            uint64_t k1[1] = {(uint32_t)lane < n ? s.keys[lane] : ~0ull};
            wave_sort_regs<1>(k1);
            if (lane < kout) emit(lane, k1[0]);
        } else if (n <= 128) {
            uint64_t k2[2];
#pragma unroll
            for (int e = 0; e < 2; e++) k2[e] = (uint32_t)(e * 64 + lane) < n ? s.keys[e * 64 + lane] : ~0ull;
            wave_sort_regs<2>(k2);
#pragma unroll
            for (int e = 0; e < 2; e++)
                if (e * 64 + lane < kout) emit(e * 64 + lane, k2[e]);
            done = 128;
        } else {
            uint64_t k4[4];
#pragma unroll
            for (int e = 0; e < 4; e++) k4[e] = (uint32_t)(e * 64 + lane) < n ? s.keys[e * 64 + lane] : ~0ull;
            wave_sort_regs<4>(k4);
#pragma unroll
            for (int e = 0; e < 4; e++)
                if (e * 64 + lane < kout) emit(e * 64 + lane, k4[e]);
            done = 256;
        }
        for (int j = done + lane; j < kout; j += 64) emit(j, ~0ull);  // j >= n: padding
        return;
    }
    const int n2 = next_pow2((int)n);
    for (int t = (int)n + tid; t < n2; t += VGPU_BLOCK) s.keys[t] = ~0ull;
    block_bitonic_sort_keys(s.keys, n2);
    for (int j = tid; j < kout; j += VGPU_BLOCK) {
        const size_t o = (size_t)q * kout + j;
        if ((uint32_t)j < n) {
            a.out_vidx[o] = (uint32_t)s.keys[j];
            a.out_dist[o] = key_dist(s.keys[j]);
        } else {
            a.out_vidx[o] = 0xffffffffu;
            a.out_dist[o] = __int_as_float(0x7f800000);
        }
    }
}

// Static table bytes of the specialisations (compile-time M, K = 256).
static size_t static_lut_bytes(const DevIndex& ix) {
    if (ix.K != 256) return 0;
    switch (ix.M) {
        case 4: case 8: case 16: case 32: case 48: case 64: return (size_t)ix.M * 256 * 4;
        default: return 0;
    }
}

size_t scan8_fast_lds_bytes(const DevIndex& ix, const ScanArgs& a) {
    size_t off[11];
    const size_t st = static_lut_bytes(ix);
    return st + fs8_layout(ix.d, ix.M, ix.K, a.P, fs8_buf(a.kk), st != 0, off);
}

template <int MT, int KT, int DS>
static void launch_fast(const DevIndex& ix, const ScanArgs& a, hipStream_t s, hipEvent_t t0,
                        hipEvent_t t1) {
    const int buf = fs8_buf(a.kk);
    size_t off[11];
    const size_t dyn = fs8_layout(ix.d, ix.M, ix.K, a.P, buf, MT > 0 && KT >= 64, off);
    auto k = scan8_fast_kernel<MT, KT, DS>;
    ensure_dyn_lds((const void*)k, dyn);
    if (t0)
        hipExtLaunchKernelGGL(k, dim3(a.nq), dim3(VGPU_BLOCK), (uint32_t)dyn, s, t0, t1, 0u, ix, a, buf);
    else
        hipLaunchKernelGGL(k, dim3(a.nq), dim3(VGPU_BLOCK), dyn, s, ix, a, buf);
}

template <int MT>
static void launch_fast_m(const DevIndex& ix, const ScanArgs& a, hipStream_t s, hipEvent_t t0,
                          hipEvent_t t1) {
    switch (ix.ds) {  // the subvector widths of the benchmark shapes
        case 2: launch_fast<MT, 256, 2>(ix, a, s, t0, t1); return;
        case 4: launch_fast<MT, 256, 4>(ix, a, s, t0, t1); return;
        case 8: launch_fast<MT, 256, 8>(ix, a, s, t0, t1); return;
        default: launch_fast<MT, 256, 0>(ix, a, s, t0, t1); return;
    }
}

void launch_scan8_fast(const DevIndex& ix, const ScanArgs& a, hipStream_t s, hipEvent_t t0, hipEvent_t t1) {
    if (a.nq <= 0) return;
    if (ix.K == 256) {
        switch (ix.M) {
            case 4: launch_fast_m<4>(ix, a, s, t0, t1); return;
            case 8: launch_fast_m<8>(ix, a, s, t0, t1); return;
            case 16: launch_fast_m<16>(ix, a, s, t0, t1); return;
            case 32: launch_fast_m<32>(ix, a, s, t0, t1); return;
            case 48: launch_fast_m<48>(ix, a, s, t0, t1); return;
            case 64: launch_fast_m<64>(ix, a, s, t0, t1); return;
            default: break;
        }
    }
    launch_fast<0, 0, 0>(ix, a, s, t0, t1);
}

}  // namespace vgpu
