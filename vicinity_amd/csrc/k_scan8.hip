// ADC scan over the probed inverted lists for byte codes (codebook_size != 16),
// one workgroup (512 threads) per query.
//
// Reference: search_approx_internal_observed src/ivf_pq/search.rs:1175-1391;
// compute_adc_table_into src/ivf_pq/pq.rs:196-266; adc_batch_256_into
// src/pq_simd.rs:330-369 (sum of LUT[m][code[m]] for m = 0..M-1 from 0.0);
// finish_top_k_by_distance search.rs:64-75.
//
// EXACT mode restates the reference arithmetic: per probed list the residual
// r = q - c and the table LUT[m][k] = sum_j (r_j - cw_j)^2 (sub, mul, add in
// order) live in LDS; each candidate sums its M entries in codebook order.
// A step takes two probed lists when both tables fit (built in one pass over
// the codebooks, scanned in one set of rounds), with the next step's residual
// elements, list ids and code rows already loading.
//
// This kernel serves EXACT mode and the queries FAST mode (k_scan8_fast.hip)
// could not prove; it writes the same rows FAST mode would have written.
#include "vgpu_device.h"
#include "vgpu_launch.h"

namespace vgpu {

// 512 threads per query: thread (t, h) = (tid % 256, tid / 256) builds
// codeword t's table entries of the codebooks m = h, h + 2, ..., so each holds
// half the codewords in registers and two workgroups fit a CU.
#define SCAN_THREADS 512
#define SCAN_WAVES (SCAN_THREADS / 64)
#define SCAN_U 1                        // candidates per thread per round
#define SCAN_ROUND (SCAN_THREADS * SCAN_U)

// Codewords a thread holds: ds (CWD < 0: exactly -CWD, CWD > 0: up to CWD)
// floats of each of its ceil(MT / 2) codebooks.
template <int MT, int CWD>
constexpr int cw_count() {
    return CWD != 0 ? (MT + 1) / 2 * (CWD > 0 ? CWD : -CWD) : 1;
}

// Probe slots kept in LDS per query; a wider probe (nprobe up to nlist) reads
// each slot's list from global memory when it is scanned.
#define SCAN_LDS_P 1024

struct TopkLds {
    uint64_t* keys;  // (distance key << 32) | vector index
    uint32_t* count;
    uint32_t* thr;   // distance key threshold: accept fkey(dist) <= thr
};

// Ascending sort of the N = SCAN_THREADS * E keys in LDS, in place.  Lane l
// of wave w holds element w * 64 E + 64 j + l in k[j]: the bitonic stages of
// strides below 64 exchange registers between lanes, those of strides 64 to
// 64 E - 1 between a thread's own registers, and only the strides of 64 E and
// up (across waves) go through LDS, two barriers each.
template <int E>
__device__ void scan_sort_keys(uint64_t* keys) {
    constexpr int N = SCAN_THREADS * E, WE = 64 * E;
    const int lane = threadIdx.x & 63, wbase = (threadIdx.x >> 6) * WE + lane;
    uint64_t k[E];
    __syncthreads();
#pragma unroll
    for (int j = 0; j < E; j++) k[j] = keys[wbase + 64 * j];
#pragma unroll
    for (int size = 2; size <= N; size <<= 1) {
#pragma unroll
        for (int stride = size >> 1; stride > 0; stride >>= 1) {
            if (stride >= WE) {
                __syncthreads();  // the previous exchange's reads are done
#pragma unroll
                for (int j = 0; j < E; j++) keys[wbase + 64 * j] = k[j];
                __syncthreads();
#pragma unroll
                for (int j = 0; j < E; j++) {
                    const int e = wbase + 64 * j;
                    const uint64_t o = keys[e ^ stride];
                    k[j] = ((e & stride) == 0) == ((e & size) == 0) ? min(o, k[j]) : max(o, k[j]);
                }
            } else if (stride >= 64) {
                const int js = stride >> 6;
#pragma unroll
                for (int j = 0; j < E; j++) {
                    const int f = j ^ js;
                    if (f > j) {
                        const bool asc = ((wbase + 64 * j) & size) == 0;
                        const uint64_t a = k[j], b = k[f];
                        k[j] = asc ? min(a, b) : max(a, b);
                        k[f] = asc ? max(a, b) : min(a, b);
                    }
                }
            } else {
#pragma unroll
                for (int j = 0; j < E; j++) {
                    const int e = wbase + 64 * j;
                    const uint64_t o = shfl_xor_u64(k[j], stride);
                    k[j] = ((e & stride) == 0) == ((e & size) == 0) ? min(o, k[j]) : max(o, k[j]);
                }
            }
        }
    }
    __syncthreads();
#pragma unroll
    for (int j = 0; j < E; j++) keys[wbase + 64 * j] = k[j];
    __syncthreads();
}

// Ascending bitonic sort of keys[0..n) in LDS (n a power of two), thread t
// taking pairs t, t + SCAN_THREADS, ...  Pair t lies in the 128-key chunk t /
// 64 for strides up to 64, and every pair of a chunk belongs to one wave, so
// such a stage waits only for its own wave when the stage before it was also
// chunk-local; the stages of strides 128 and up, and the stage after each,
// wait for the block.
__device__ void scan_sort_keys_lds(uint64_t* keys, int n) {
    bool prev_wide = true;  // the caller's writes: the first stage waits for the block
    for (int size = 2; size <= n; size <<= 1) {
        for (int stride = size >> 1; stride > 0; stride >>= 1) {
            const bool wide = stride >= 128;
            if (wide || prev_wide) {
                __syncthreads();
            } else {
                __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
                __builtin_amdgcn_wave_barrier();
            }
            prev_wide = wide;
            for (int t = threadIdx.x; t < (n >> 1); t += SCAN_THREADS) {
                const int i = 2 * t - (t & (stride - 1)), j = i + stride;
                const bool asc = (i & size) == 0;
                const uint64_t a = keys[i], b = keys[j];
                if ((a > b) == asc) {
                    keys[i] = b;
                    keys[j] = a;
                }
            }
        }
    }
    __syncthreads();
}

// Sort the buffer and keep the best `keep` entries; later candidates must beat
// the keep-th distance.  All threads call it.  The keys are unique (vector
// index in the low word), so the kept set is the same whatever order the
// candidates arrived in.  REG: the register sort (a final flush, when the
// caller holds no other large register state), else the LDS sort.
template <bool REG>
__device__ void topk_flush(TopkLds& t, int keep) {
    __syncthreads();
    const int n = (int)*t.count;
    const int n2 = next_pow2(n > 0 ? n : 1);
    const int N = n2 < SCAN_THREADS ? SCAN_THREADS : n2;  // the buffer holds at least 2 x SCAN_THREADS
    for (int i = n + threadIdx.x; i < N; i += SCAN_THREADS) t.keys[i] = ~0ull;
    if (REG && N == SCAN_THREADS) scan_sort_keys<1>(t.keys);
    else if (REG && N == 2 * SCAN_THREADS) scan_sort_keys<2>(t.keys);
    else scan_sort_keys_lds(t.keys, N);
    if (threadIdx.x == 0) {
        if (n >= keep) {
            *t.thr = (uint32_t)(t.keys[keep - 1] >> 32);
            *t.count = (uint32_t)keep;
        }
    }
    __syncthreads();
}

// Four table lookups from one code word, in codebook order.
template <int KT>
__device__ __forceinline__ float add4(float s, uint32_t w, const float* lut, int K) {
    const int k = KT > 0 ? KT : K;
    s += lut[w & 0xffu];
    s += lut[k + ((w >> 8) & 0xffu)];
    s += lut[2 * k + ((w >> 16) & 0xffu)];
    s += lut[3 * k + (w >> 24)];
    return s;
}

// s + sum_{m=0}^{M-1} lut[m*K + row[m]], m in order.
template <int MT, int KT>
__device__ __forceinline__ float adc_sum(const uint8_t* __restrict__ row,
                                         const float* __restrict__ lut, int M, int K, float s) {
    const int k = KT > 0 ? KT : K;
    if constexpr (MT > 0 && MT % 16 == 0) {
        const uint4* p = reinterpret_cast<const uint4*>(row);
#pragma unroll
        for (int v = 0; v < MT / 16; v++) {
            uint4 x = p[v];
            s = add4<KT>(s, x.x, lut + (16 * v + 0) * k, K);
            s = add4<KT>(s, x.y, lut + (16 * v + 4) * k, K);
            s = add4<KT>(s, x.z, lut + (16 * v + 8) * k, K);
            s = add4<KT>(s, x.w, lut + (16 * v + 12) * k, K);
        }
    } else if constexpr (MT == 8) {
        uint2 x = *reinterpret_cast<const uint2*>(row);
        s = add4<KT>(s, x.x, lut, K);
        s = add4<KT>(s, x.y, lut + 4 * k, K);
    } else if constexpr (MT == 4) {
        uint32_t x = *reinterpret_cast<const uint32_t*>(row);
        s = add4<KT>(s, x, lut, K);
    } else {
        for (int m = 0; m < M; m++) s += lut[m * k + row[m]];
    }
    return s;
}

struct ScanLds {
    float* qs;      // [d]
    float* rsd;     // [d] EXACT residual
    float* lut;     // [M*K]
    float* rsd2;    // second residual and table (two lists per step), else rsd / lut
    float* lut2;
    int G;          // lists per step, 1 or 2
    uint32_t* lbeg; // [P]
    uint32_t* llen; // [P]
    uint32_t* lid;  // [P]
    uint32_t* pref; // [P+1]
    float* term0;   // [P]
    TopkLds tk;
    uint32_t* misc; // [4 + 2 SCAN_WAVES]
    uint4* cst;     // [SCAN_THREADS] code row of the thread's first-round entry (M <= 16)
    uint32_t* vst;  // [SCAN_THREADS] its vector index
};

// The buffer count as every thread of the block knows it, without reading
// the shared counter (which a faster wave may already have advanced): each
// round's appends are counted per wave into misc[4 + 8 par + wave] before the
// round's closing barrier and summed by every thread after it (par alternates,
// so a wave one round ahead never overwrites counts still being read).
struct TopkCnt {
    uint32_t n = 0;
    uint32_t par = 0;
};

__host__ __device__ inline size_t align16(size_t x) { return (x + 15) & ~(size_t)15; }

__host__ __device__ inline int scan_buf(int kk) {
    int need = kk + SCAN_ROUND;
    int b = 1;
    while (b < need) b <<= 1;
    return b;
}

// G residuals and tables (G lists scanned per step).
__host__ __device__ inline size_t scan_lds_layout(int d, int M, int K, int P, int buf, int G,
                                                  size_t* off /* 16 */) {
    size_t o = 0;
    off[0] = o; o = align16(o + (size_t)d * 4);          // qs
    off[1] = o; o = align16(o + (size_t)d * 4);          // rsd
    off[14] = G == 2 ? o : off[1]; o = G == 2 ? align16(o + (size_t)d * 4) : o;          // rsd2
    off[2] = o; o = align16(o + (size_t)M * K * 4);      // lut
    off[15] = G == 2 ? o : off[2]; o = G == 2 ? align16(o + (size_t)M * K * 4) : o;      // lut2
    off[3] = o; o = align16(o + (size_t)P * 4);          // lbeg
    off[4] = o; o = align16(o + (size_t)P * 4);          // llen
    off[5] = o; o = align16(o + (size_t)P * 4);          // lid
    off[6] = o; o = align16(o + (size_t)(P + 1) * 4);    // pref
    off[7] = o; o = align16(o + (size_t)P * 4);          // term0
    off[8] = o; o = align16(o + (size_t)buf * 8);        // keys
    off[11] = o; o = align16(o + 4 * (4 + 2 * SCAN_WAVES)); // misc: count, thr, 2 x 8 round counts
    off[12] = o; o = align16(o + (size_t)SCAN_THREADS * 16);  // cst
    off[13] = o; o = align16(o + (size_t)SCAN_THREADS * 4);   // vst
    return o;
}

// Two lists per step when their tables fit in half a CU's 160 KiB of LDS (so
// two workgroups still share a CU), else one.
#define SCAN_PAIR_LDS (80 * 1024)
__host__ __device__ inline int scan_groups(int d, int M, int K, int P, int buf) {
    size_t off[16];
    return scan_lds_layout(d, M, K, P, buf, 2, off) <= SCAN_PAIR_LDS ? 2 : 1;
}

__device__ inline ScanLds carve(char* smem, int d, int M, int K, int P, int buf) {
    size_t off[16];
    ScanLds s;
    s.G = scan_groups(d, M, K, P, buf);
    scan_lds_layout(d, M, K, P, buf, s.G, off);
    s.qs = (float*)(smem + off[0]);
    s.rsd = (float*)(smem + off[1]);
    s.lut = (float*)(smem + off[2]);
    s.rsd2 = (float*)(smem + off[14]);
    s.lut2 = (float*)(smem + off[15]);
    s.lbeg = (uint32_t*)(smem + off[3]);
    s.llen = (uint32_t*)(smem + off[4]);
    s.lid = (uint32_t*)(smem + off[5]);
    s.pref = (uint32_t*)(smem + off[6]);
    s.term0 = (float*)(smem + off[7]);
    s.tk.keys = (uint64_t*)(smem + off[8]);
    s.misc = (uint32_t*)(smem + off[11]);
    s.cst = (uint4*)(smem + off[12]);
    s.vst = (uint32_t*)(smem + off[13]);
    s.tk.count = s.misc;
    s.tk.thr = s.misc + 1;
    return s;
}

// Common prologue: query vector and probed list ranges into LDS (the ranges
// only for at most SCAN_LDS_P probes: wider probes are read per slot).
__device__ inline void load_query_and_lists(const DevIndex& ix, const ScanArgs& a, ScanLds& s,
                                            int q) {
    const int tid = threadIdx.x, d = ix.d, P = a.P > SCAN_LDS_P ? 0 : a.P;
    for (int j = tid; j < d; j += SCAN_THREADS) s.qs[j] = a.qn[(size_t)q * d + j];
    for (int p = tid; p < P; p += SCAN_THREADS) {
        uint32_t l = a.probe[(size_t)q * P + p];
        if (l >= (uint32_t)ix.L) {  // no such list: scanned as empty
            s.lid[p] = 0;
            s.lbeg[p] = 0;
            s.llen[p] = 0;
            continue;
        }
        uint32_t b = ix.offsets[l];
        s.lid[p] = l;
        s.lbeg[p] = b;
        s.llen[p] = ix.offsets[l + 1] - b;
    }
    if (tid == 0) {
        *s.tk.count = 0;
        *s.tk.thr = 0xffffffffu;
    }
    __syncthreads();
    if (tid == 0) {
        uint32_t acc = 0;
        s.pref[0] = 0;
        for (int p = 0; p < P; p++) {
            acc += s.llen[p];
            s.pref[p + 1] = acc;
        }
    }
}

// Write the first kout sorted entries, padded (scan_emit).
__device__ inline void write_out(const ScanArgs& a, ScanLds& s, int q, int n) {
    for (int j = threadIdx.x; j < a.kout; j += SCAN_THREADS) scan_emit(a, q, j, s.tk.keys[j], j < n);
}

// Probed list l (slot p, entries beg .. beg + len - 1) with the reference
// arithmetic, in three steps: the residual r = q - c (search.rs:1242-1245;
// with OPQ the rotated residual R r, precomputed per slot in a.rres) into
// rsd; the table LUT[m][k] = sum_j (r_j - cw_j)^2 (pq.rs:232-251; ds == 1
// gives 0 + diff*diff == diff*diff) from rsd into lut; then each entry's M
// entries summed in codebook order (pq.rs:272-279).  With FILT only the
// entries whose category byte equals cq are candidates (filtering/mod.rs:151-
// 153, 214-218).  Every thread of the block calls each step.
__device__ inline void stage_residual(const DevIndex& ix, const ScanArgs& a, const ScanLds& s, float* rsd,
                                      uint32_t l, int q, int p) {
    const int tid = threadIdx.x, d = ix.d;
    if (a.rres) {  // OPQ: R (q - c), formed by the rotation kernel (opq.rs:120-123)
        const float* rr = a.rres + ((size_t)q * a.P + p) * d;
        for (int j = tid; j < d; j += SCAN_THREADS) rsd[j] = rr[j];
    } else {
        const float* c = ix.centroids + (size_t)l * d;
        for (int j = tid; j < d; j += SCAN_THREADS) rsd[j] = s.qs[j] - c[j];
    }
}

template <int MT, int KT, int CWD>
__device__ inline void build_table(const DevIndex& ix, const float* rsd, float* lut,
                                   const float (&cw)[cw_count<MT, CWD>()]) {
    const int tid = threadIdx.x;
    const int M = MT > 0 ? MT : ix.M, K = KT > 0 ? KT : ix.K, ds = ix.ds;
    const int t = tid & 255, h = (tid >> 8) & 1;  // codeword, codebook parity (wave-uniform)
    if constexpr (CWD < 0) {  // ds == W: codewords in registers, the next slice read ahead
        constexpr int W = -CWD;
        static_assert(MT % 2 == 0 && KT == 256, "codebook pairs of ksub 256");
        // one LDS base each, the codebook in the immediate offset: the slice
        // of codebook m = 2 i + h at rr[2 i W], entry (m, t) at lw[512 i]
        const float* rr = rsd + h * W;
        float* lw = lut + (tid & 511);
        float rc[W], rn[W];
#pragma unroll
        for (int j = 0; j < W; j++) rc[j] = rr[j];
#pragma unroll
        for (int i = 0; i < MT / 2; i++) {
            if (i + 1 < MT / 2) {
#pragma unroll
                for (int j = 0; j < W; j++) rn[j] = rr[(2 * i + 2) * W + j];
            }
            float acc = 0.0f;
#pragma unroll
            for (int j = 0; j < W; j++) {
                float diff = rc[j] - cw[i * W + j];
                acc += diff * diff;
            }
            lw[512 * i] = acc;
#pragma unroll
            for (int j = 0; j < W; j++) rc[j] = rn[j];
            // two slices live at a time: the compiler may not hoist further reads
            __builtin_amdgcn_sched_barrier(0);
        }
    } else if constexpr (CWD > 0) {  // ds < CWD: codewords in registers, guarded
        constexpr int W = CWD;
        const int dsx = ds;
#pragma unroll
        for (int i = 0; i < (MT + 1) / 2; i++) {
            const int m = 2 * i + h;
            float acc = 0.0f;
#pragma unroll
            for (int j = 0; j < W; j++) {
                if (j < dsx && m < MT) {
                    float diff = rsd[m * dsx + j] - cw[i * W + j];
                    acc += diff * diff;
                }
            }
            if (m < MT) lut[m * 256 + t] = acc;
            // one codebook's residual slice live at a time (hoisting every
            // LDS read ahead of the arithmetic would double the registers)
            __builtin_amdgcn_sched_barrier(0);
        }
    } else {
        for (int e = tid; e < M * K; e += SCAN_THREADS) {
            const int m = e / K;
            const float* cwp = ix.codebooks + (size_t)e * ds;
            float acc = 0.0f;
            for (int j = 0; j < ds; j++) {
                float diff = rsd[m * ds + j] - cwp[j];
                acc += diff * diff;
            }
            lut[e] = acc;
        }
    }
}

// The tables of a step: slot A's from s.rsd into s.lut and, when two, slot
// B's from s.rsd2 into s.lut2.  With ds == -CWD (codewords in registers) the
// two tables are built in one pass over the codebooks, each codeword register
// serving both, and the second residual and table sit at fixed offsets from
// the first (the layout places them back to back), so one LDS address serves
// both.
template <int MT, int KT, int CWD>
__device__ inline void build_tables(const DevIndex& ix, const ScanLds& s, bool two,
                                    const float (&cw)[cw_count<MT, CWD>()]) {
    if constexpr (CWD < 0 && KT == 256) {
        constexpr int W = -CWD;
        constexpr int RS = (MT * W + 3) & ~3;  // floats from rsd to rsd2
        constexpr int LS = MT * KT;            // floats from lut to lut2
        const int tid = threadIdx.x, h = (tid >> 8) & 1;
        if (!two) {
            build_table<MT, KT, CWD>(ix, s.rsd, s.lut, cw);
            return;
        }
        const float* rr = s.rsd + h * W;  // as in build_table, both tables off one base
        float* lw = s.lut + (tid & 511);
#pragma unroll
        for (int i = 0; i < MT / 2; i++) {
            float ra[W], rb[W];
#pragma unroll
            for (int j = 0; j < W; j++) {
                ra[j] = rr[2 * i * W + j];
                rb[j] = rr[RS + 2 * i * W + j];
            }
            float acc_a = 0.0f, acc_b = 0.0f;
#pragma unroll
            for (int j = 0; j < W; j++) {
                const float da = ra[j] - cw[i * W + j], db = rb[j] - cw[i * W + j];
                acc_a += da * da;
                acc_b += db * db;
            }
            lw[512 * i] = acc_a;
            lw[LS + 512 * i] = acc_b;
            __builtin_amdgcn_sched_barrier(0);
        }
    } else {
        build_table<MT, KT, CWD>(ix, s.rsd, s.lut, cw);
        if (two) build_table<MT, KT, CWD>(ix, s.rsd2, s.lut2, cw);
    }
}

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));

// Code rows of at most 16 bytes are read one slot ahead (pre_words words).
template <int MT>
constexpr int pre_words() {
    return (MT == 4 || MT == 8 || MT == 16) ? MT / 4 : 0;
}

// s + the table entries of the code row held in words w, in codebook order
// (the sum adc_sum forms from the row in memory).
template <int MT, int KT>
__device__ __forceinline__ float adc_words(const uint4& w, const float* __restrict__ lut, int K, float s) {
    const int k = KT > 0 ? KT : K;
    s = add4<KT>(s, w.x, lut, K);
    if constexpr (MT >= 8) s = add4<KT>(s, w.y, lut + 4 * k, K);
    if constexpr (MT >= 16) {
        s = add4<KT>(s, w.z, lut + 8 * k, K);
        s = add4<KT>(s, w.w, lut + 12 * k, K);
    }
    return s;
}

// A probe slot: its index, list, first entry and length (uniform).
struct SlotRef {
    int p;
    uint32_t l, beg, len;
};

// The loads of the next step's slots A and B (B.len == 0 when there is no
// B), issued while the current step is scanned: element tid of each residual
// source (the centroid row, or with OPQ the rotated residual), and the vector
// index and (M <= 16) code row of entry tid of A's list followed by B's,
// which the step's first round scores.
template <int MT>
struct PairPre {
    float ca, cb;
    uint32_t vid;
    uint4 w;
};

template <int MT>
__device__ inline void pair_prefetch(const DevIndex& ix, const ScanArgs& a, int q, int P, const SlotRef& A,
                                     const SlotRef& B, PairPre<MT>& pr) {
    // Raw buffer loads over the slots' own ranges: uniform bases, 32-bit lane
    // offsets, and lanes past a range read zeros without touching memory.
    const uint32_t tid = threadIdx.x, d = (uint32_t)ix.d;
    auto resid = [&](const SlotRef& X) {
        const float* src = a.rres ? a.rres + ((size_t)q * a.P + X.p) * d : ix.centroids + (size_t)X.l * d;
        const __amdgpu_buffer_rsrc_t r =
            __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(src), (short)0, (int)(d * 4u), 0x00020000);
        return __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(r, tid * 4u, 0u, 0));
    };
    pr.ca = resid(A);
    pr.cb = B.p < P ? resid(B) : 0.0f;
    pr.vid = 0u;
    pr.w = make_uint4(0u, 0u, 0u, 0u);
    auto entry = [&](const SlotRef& X, uint32_t e) {
        const __amdgpu_buffer_rsrc_t ri = __builtin_amdgcn_make_buffer_rsrc(
            const_cast<uint32_t*>(ix.list_ids + X.beg), (short)0, (int)(X.len * 4u), 0x00020000);
        pr.vid = __builtin_amdgcn_raw_buffer_load_b32(ri, e * 4u, 0u, 0);
        if constexpr (pre_words<MT>() > 0) {
            const __amdgpu_buffer_rsrc_t rw = __builtin_amdgcn_make_buffer_rsrc(
                const_cast<uint8_t*>(ix.codes + (size_t)X.beg * MT), (short)0, (int)(X.len * (uint32_t)MT),
                0x00020000);
            if constexpr (pre_words<MT>() == 4) {
                const u32x4 x = __builtin_amdgcn_raw_buffer_load_b128(rw, e * 16u, 0u, 0);
                pr.w = make_uint4(x[0], x[1], x[2], x[3]);
            } else if constexpr (pre_words<MT>() == 2) {
                const u32x2 x = __builtin_amdgcn_raw_buffer_load_b64(rw, e * 8u, 0u, 0);
                pr.w.x = x[0];
                pr.w.y = x[1];
            } else {
                pr.w.x = __builtin_amdgcn_raw_buffer_load_b32(rw, e * 4u, 0u, 0);
            }
        }
    };
    if (tid < A.len) entry(A, tid);
    else if (tid - A.len < B.len) entry(B, tid - A.len);
}

// The entries of list A, then of list B (B.len == 0: none), each against its
// own table (lut_a, lut_b); a block barrier ends every round.  The flush
// decision uses the count every thread holds in tc, so it is the same in every
// wave.  PRE: the first round takes each thread's code row (M <= 16) and
// vector index from s.cst / s.vst, staged by the thread itself from its
// pair_prefetch loads.
template <int MT, int KT, bool FILT, bool PRE = false>
__device__ inline void scan_entries(const DevIndex& ix, const ScanArgs& a, ScanLds& s, int buf, const SlotRef& A,
                                    const float* lut_a, const SlotRef& B, const float* lut_b,
                                    const uint8_t* __restrict__ ecat, uint8_t cq, TopkCnt& tc) {
    const int tid = threadIdx.x;
    const int M = MT > 0 ? MT : ix.M, K = KT > 0 ? KT : ix.K;
    static_assert(!PRE || SCAN_U == 1, "one staged entry per thread");
    const uint32_t len = A.len + B.len;
    for (uint32_t base = 0; base < len; base += SCAN_ROUND) {
        if (tc.n > (uint32_t)(buf - SCAN_ROUND)) {
            topk_flush<false>(s.tk, a.kk);
            tc.n = tc.n >= (uint32_t)a.kk ? (uint32_t)a.kk : tc.n;  // the flush keeps kk when it has them
        }
        const uint32_t thr = *s.tk.thr;
        uint32_t wn = 0;  // this wave's appends in the round
#pragma unroll
        for (int u = 0; u < SCAN_U; u++) {
            uint32_t i = base + u * SCAN_THREADS + tid;
            bool take = false;
            uint32_t fk = 0, pos = 0;
            const bool staged = PRE && base == 0;  // uniform
            const bool in_a = i < A.len;
            if (i < len) {
                pos = in_a ? A.beg + i : B.beg + (i - A.len);
                if (!FILT || ecat[pos] == cq) {
                    const float* lut = in_a ? lut_a : lut_b;
                    float dist;
                    if (staged && pre_words<MT>() > 0) dist = adc_words<MT, KT>(s.cst[tid], lut, K, 0.0f);
                    else dist = adc_sum<MT, KT>(ix.codes + (size_t)pos * M, lut, M, K, 0.0f);
                    fk = fkey(dist);
                    take = fk <= thr;
                }
            }
            wn += (uint32_t)__popcll(__ballot(take));
            const int slot = wave_append_slot(take, s.tk.count);
            if (take) s.tk.keys[slot] = ((uint64_t)fk << 32) | (staged ? s.vst[tid] : ix.list_ids[pos]);
        }
        if ((tid & 63) == 0) s.misc[4 + SCAN_WAVES * tc.par + (tid >> 6)] = wn;
        __syncthreads();
#pragma unroll
        for (int w = 0; w < SCAN_WAVES; w++) tc.n += s.misc[4 + SCAN_WAVES * tc.par + w];
        tc.par ^= 1u;
    }
}

template <int MT, int KT, bool FILT, int CWD>
__device__ inline void scan_list(const DevIndex& ix, const ScanArgs& a, ScanLds& s, int buf,
                                 uint32_t l, uint32_t beg, uint32_t len, int q, int p,
                                 const uint8_t* __restrict__ ecat, uint8_t cq,
                                 const float (&cw)[cw_count<MT, CWD>()], TopkCnt& tc) {
    stage_residual(ix, a, s, s.rsd, l, q, p);
    __syncthreads();
    build_table<MT, KT, CWD>(ix, s.rsd, s.lut, cw);
    __syncthreads();
    const SlotRef A{p, l, beg, len}, none{0, 0u, 0u, 0u};
    scan_entries<MT, KT, FILT>(ix, a, s, buf, A, s.lut, none, s.lut, ecat, cq, tc);
}

// Codeword t = tid % 256 of the codebooks h, h + 2, ... (h = tid / 256) into
// registers (ksub 256): CWD > 0 holds ds <= CWD floats per codeword, CWD < 0
// exactly ds = -CWD.  The per-list tables then read no codebook memory.
template <int MT, int CWD>
__device__ inline void load_codewords(const DevIndex& ix, float (&cw)[cw_count<MT, CWD>()]) {
    if constexpr (CWD != 0) {
        constexpr int W = CWD > 0 ? CWD : -CWD;
        const int t = threadIdx.x & 255, h = (threadIdx.x >> 8) & 1, ds = CWD > 0 ? ix.ds : W;
#pragma unroll
        for (int i = 0; i < (MT + 1) / 2; i++) {
            const int m = 2 * i + h;
            const float* src = ix.codebooks + ((size_t)(m < MT ? m : 0) * 256 + t) * ds;
#pragma unroll
            for (int j = 0; j < W; j++) cw[i * W + j] = j < ds && m < MT ? src[j] : 0.0f;
        }
    }
}

// One query with the reference arithmetic; every thread of the block calls it.
template <int MT, int KT, int CWD>
__device__ void exact_query(const DevIndex& ix, const ScanArgs& a, int buf, char* smem, int q,
                            const float (&cw)[cw_count<MT, CWD>()]) {
    const int tid = threadIdx.x;
    // with ds == -CWD the dimension is MT * ds: compile-time, and so are the
    // LDS offsets of the query, residuals and tables
    const int d = CWD < 0 ? MT * -CWD : ix.d, M = MT > 0 ? MT : ix.M, K = KT > 0 ? KT : ix.K, P = a.P;
    const bool wide = P > SCAN_LDS_P;
    ScanLds s = carve(smem, d, M, K, wide ? 0 : P, buf);
    load_query_and_lists(ix, a, s, q);
    // list, begin and length of probe slot p (the same for every thread)
    auto slot = [&](int p, uint32_t& l, uint32_t& beg, uint32_t& len) {
        if (wide) {
            l = a.probe[(size_t)q * P + p];
            const bool ok = l < (uint32_t)ix.L;
            beg = ok ? ix.offsets[l] : 0u;
            len = ok ? ix.offsets[l + 1] - beg : 0u;
        } else {  // uniform: held in scalar registers
            l = __builtin_amdgcn_readfirstlane(s.lid[p]);
            beg = __builtin_amdgcn_readfirstlane(s.lbeg[p]);
            len = __builtin_amdgcn_readfirstlane(s.llen[p]);
        }
    };
    uint32_t total = 0;
    // the first non-empty slot at or after `from` ({P, 0, 0, 0} when there is none)
    auto next = [&](int from, SlotRef& x) {
        x = SlotRef{P, 0u, 0u, 0u};
        for (int pn = from; pn < P; pn++) {
            uint32_t l, beg, len;
            slot(pn, l, beg, len);
            total += len;
            if (len != 0u) {
                x = SlotRef{pn, l, beg, len};
                break;
            }
        }
    };
    // the next step's slots: A, and B after it when two lists fit per step
    auto step = [&](int from, SlotRef& x, SlotRef& y) {
        next(from, x);
        y = SlotRef{P, 0u, 0u, 0u};
        if (s.G == 2 && x.p < P) next(x.p + 1, y);
    };
    // the residual of slot x into r, from the element tid loaded a step ahead
    auto stage = [&](const SlotRef& x, float c, float* r) {
        if (tid < d) r[tid] = a.rres ? c : s.qs[tid] - c;
        for (int j = tid + SCAN_THREADS; j < d; j += SCAN_THREADS)
            r[j] = a.rres ? a.rres[((size_t)q * P + x.p) * d + j] : s.qs[j] - ix.centroids[(size_t)x.l * d + j];
    };
    TopkCnt tc;
    PairPre<MT> pre;
    SlotRef A, B;
    step(0, A, B);
    if (A.p < P) pair_prefetch<MT>(ix, a, q, P, A, B, pre);
    // Each step: the residuals from the elements loaded a step earlier, the
    // loads of the next step issued, the tables, then the entries of both
    // lists (the first round from the staged code rows).
    while (A.p < P) {
        SlotRef nA, nB;
        step((B.p < P ? B.p : A.p) + 1, nA, nB);
        // no barrier: the last round of the previous step ended with one, after
        // every read of its residuals, tables and staged rows
        stage(A, pre.ca, s.rsd);
        if (B.p < P) stage(B, pre.cb, s.rsd2);
        if ((uint32_t)tid < A.len + B.len) {  // read back by this thread only
            if constexpr (pre_words<MT>() > 0) s.cst[tid] = pre.w;
            s.vst[tid] = pre.vid;
        }
        if (nA.p < P) pair_prefetch<MT>(ix, a, q, P, nA, nB, pre);
        __syncthreads();
        build_tables<MT, KT, CWD>(ix, s, B.p < P, cw);
        __syncthreads();
        scan_entries<MT, KT, false, true>(ix, a, s, buf, A, s.lut, B, s.lut2, nullptr, 0, tc);
        A = nA;
        B = nB;
    }
    topk_flush<true>(s.tk, a.kk);
    const int n = (int)*s.tk.count;
    if (tid == 0 && !a.only_flagged) {
        uint32_t* st = a.qstat + (size_t)q * QSTAT_WORDS;
        st[0] = total;
        st[1] = st[2] = st[3] = 0u;
    }
    write_out(a, s, q, n < a.kout ? n : a.kout);
}

// search_with_filter (search.rs:1407-1549), one query per workgroup: the
// query's lists in slot order (the probed lists carrying its category, then,
// when it was widened, every other list carrying it; slots >= L are padding),
// scored like EXACT mode, candidates restricted to the entries whose category
// is want[q].  The list bounds are read from global memory per slot, so the
// list count is not bounded by LDS (a widened query takes every list).
template <int MT, int KT, int CWD>
__global__ __launch_bounds__(SCAN_THREADS, 4) void scan8_filtered_kernel(DevIndex ix, ScanArgs a, int buf,
                                                             const uint8_t* __restrict__ ecat,
                                                             const uint8_t* __restrict__ want) {
    extern __shared__ __align__(16) char smem[];
    const int q = blockIdx.x;
    if (q >= a.nq) return;
    const int tid = threadIdx.x;
    const int d = ix.d, M = MT > 0 ? MT : ix.M, K = KT > 0 ? KT : ix.K, P = a.P;
    ScanLds s = carve(smem, d, M, K, 0, buf);
    float cw[cw_count<MT, CWD>()];
    load_codewords<MT, CWD>(ix, cw);
    for (int j = tid; j < d; j += SCAN_THREADS) s.qs[j] = a.qn[(size_t)q * d + j];
    if (tid == 0) {
        *s.tk.count = 0;
        *s.tk.thr = 0xffffffffu;
    }
    const uint8_t cq = want[q];
    TopkCnt tc;
    for (int p = 0; p < P; p++) {
        __syncthreads();
        const uint32_t l = a.probe[(size_t)q * P + p];  // the same for every thread
        if (l >= (uint32_t)ix.L) continue;
        const uint32_t beg = ix.offsets[l], len = ix.offsets[l + 1] - beg;
        if (len == 0) continue;
        scan_list<MT, KT, true, CWD>(ix, a, s, buf, l, beg, len, q, p, ecat, cq, cw, tc);
    }
    topk_flush<true>(s.tk, a.kk);
    const int n = (int)*s.tk.count;
    write_out(a, s, q, n < a.kout ? n : a.kout);
}

// FL = false: every query of the batch, block q taking query q.  FL = true:
// the flagged queries the FAST kernel listed before this launch, the blocks
// striding over the list.  Two kernels, each with one call site of the query
// body: a loop over queries in the whole-batch kernel would keep the body's
// per-lane addresses live across it (they are loop-invariant) and spill them
// to scratch in every workgroup.
template <int MT, int KT, int CWD, bool FL>
__global__ __launch_bounds__(SCAN_THREADS, 4) void scan8_exact_kernel(DevIndex ix, ScanArgs a, int buf) {
    extern __shared__ __align__(16) char smem[];
    float cw[cw_count<MT, CWD>()];  // the same for every query
    if constexpr (!FL) {
        if (blockIdx.x >= (uint32_t)a.nq) return;
        load_codewords<MT, CWD>(ix, cw);
        exact_query<MT, KT, CWD>(ix, a, buf, smem, (int)blockIdx.x, cw);
    } else {
        const uint32_t nf = *a.flag_count;
        if (blockIdx.x >= nf) return;
        load_codewords<MT, CWD>(ix, cw);
        for (uint32_t fi = blockIdx.x; fi < nf; fi += gridDim.x) {
            __syncthreads();
            exact_query<MT, KT, CWD>(ix, a, buf, smem, (int)a.flag_list[fi], cw);
        }
    }
}

// Codewords held per thread: ksub 256 with a fixed codebook count and
// d <= 128 (M * ds floats per thread); 0 = read the codebooks per list.  The
// kernels take -W when ds is exactly W = cw_regs, 3 cw_regs / 4, cw_regs / 2 or
// cw_regs / 4 (W >= 2; d 128, 96, 64, 32: compile-time d, no guards), cw_regs
// for other ds below it.  At
// d 64 the guarded variant took 2.25x (16 codebooks) and 1.57x (32) the time
// of the exact-width one: its codeword guards, and 56 to 136 bytes per lane of
// spills.
template <int MT, int KT>
constexpr int cw_regs() {
    return (KT == 256 && MT > 0 && MT <= 64) ? 128 / MT : 0;
}

// The codeword width parameter for a run-time ds: -W, CWD, or 0 (see cw_regs),
// as the kernel template `K` instantiated at it.
template <int CWD, typename Fn, typename K>
static Fn cw_pick(int ds, K kern) {
    Fn f = kern(std::integral_constant<int, 0>{});
    if constexpr (CWD > 0) {
        if (ds == CWD) f = kern(std::integral_constant<int, -CWD>{});
        else if (ds < CWD) f = kern(std::integral_constant<int, CWD>{});
        if constexpr (CWD >= 4)
            if (ds == CWD / 2) f = kern(std::integral_constant<int, -(CWD / 2)>{});
        if constexpr (CWD >= 8)
            if (ds == CWD / 4) f = kern(std::integral_constant<int, -(CWD / 4)>{});
        if constexpr (CWD >= 4)
            if (ds == 3 * CWD / 4) f = kern(std::integral_constant<int, -(3 * CWD / 4)>{});
    }
    return f;
}

size_t scan8_lds_bytes(const DevIndex& ix, const ScanArgs& a) {
    size_t off[16];
    const int P = a.P > SCAN_LDS_P ? 0 : a.P, buf = scan_buf(a.kk);
    return scan_lds_layout(ix.d, ix.M, ix.K, P, buf, scan_groups(ix.d, ix.M, ix.K, P, buf), off);
}

template <int MT, int KT>
static void launch_mk(const DevIndex& ix, const ScanArgs& a, hipStream_t s) {
    int buf = scan_buf(a.kk);
    size_t lds = scan8_lds_bytes(ix, a);
    constexpr int CWD = cw_regs<MT, KT>();
    auto pick = [&](auto fl) {
        constexpr bool FL = decltype(fl)::value;
        using Fn = void (*)(DevIndex, ScanArgs, int);
        return cw_pick<CWD, Fn>(ix.ds, [](auto w) -> Fn {
            return scan8_exact_kernel<MT, KT, decltype(w)::value, FL>;
        });
    };
    auto k = a.only_flagged ? pick(std::true_type{}) : pick(std::false_type{});
    ensure_dyn_lds((const void*)k, lds);
    // Flagged queries: a small grid walks the list the FAST kernel wrote.
    // flagged queries are rare: a small grid keeps the usual empty launch cheap
    const int grid = a.only_flagged ? (a.nq < 64 ? a.nq : 64) : a.nq;
    hipLaunchKernelGGL(k, dim3(grid), dim3(SCAN_THREADS), lds, s, ix, a, buf);
}

template <int KT>
static void launch_k(const DevIndex& ix, const ScanArgs& a, hipStream_t s) {
    switch (ix.M) {
        case 4: launch_mk<4, KT>(ix, a, s); break;
        case 8: launch_mk<8, KT>(ix, a, s); break;
        case 16: launch_mk<16, KT>(ix, a, s); break;
        case 32: launch_mk<32, KT>(ix, a, s); break;
        case 48: launch_mk<48, KT>(ix, a, s); break;
        case 64: launch_mk<64, KT>(ix, a, s); break;
        default: launch_mk<0, KT>(ix, a, s); break;
    }
}

void launch_scan8_exact(const DevIndex& ix, const ScanArgs& a, hipStream_t s) {
    if (a.nq <= 0) return;
    if (ix.K == 256) launch_k<256>(ix, a, s);
    else launch_k<0>(ix, a, s);
}

template <int MT, int KT>
static void launch_filtered_mk(const DevIndex& ix, const ScanArgs& a, const uint8_t* ecat,
                               const uint8_t* want, hipStream_t s) {
    const int buf = scan_buf(a.kk);
    size_t off[16];
    const size_t lds = scan_lds_layout(ix.d, ix.M, ix.K, 0, buf, scan_groups(ix.d, ix.M, ix.K, 0, buf), off);
    constexpr int CWD = cw_regs<MT, KT>();
    using Fn = decltype(&scan8_filtered_kernel<MT, KT, 0>);
    auto k = cw_pick<CWD, Fn>(ix.ds, [](auto w) -> Fn { return scan8_filtered_kernel<MT, KT, decltype(w)::value>; });
    ensure_dyn_lds((const void*)k, lds);
    hipLaunchKernelGGL(k, dim3(a.nq), dim3(SCAN_THREADS), lds, s, ix, a, buf, ecat, want);
}

template <int KT>
static void launch_filtered_k(const DevIndex& ix, const ScanArgs& a, const uint8_t* ecat,
                              const uint8_t* want, hipStream_t s) {
    switch (ix.M) {
        case 4: launch_filtered_mk<4, KT>(ix, a, ecat, want, s); break;
        case 8: launch_filtered_mk<8, KT>(ix, a, ecat, want, s); break;
        case 16: launch_filtered_mk<16, KT>(ix, a, ecat, want, s); break;
        case 32: launch_filtered_mk<32, KT>(ix, a, ecat, want, s); break;
        case 48: launch_filtered_mk<48, KT>(ix, a, ecat, want, s); break;
        case 64: launch_filtered_mk<64, KT>(ix, a, ecat, want, s); break;
        default: launch_filtered_mk<0, KT>(ix, a, ecat, want, s); break;
    }
}

void launch_scan8_filtered(const DevIndex& ix, const ScanArgs& a, const uint8_t* ecat,
                           const uint8_t* want, hipStream_t s) {
    if (a.nq <= 0) return;
    if (ix.K == 256) launch_filtered_k<256>(ix, a, ecat, want, s);
    else launch_filtered_k<0>(ix, a, ecat, want, s);
}

}  // namespace vgpu
