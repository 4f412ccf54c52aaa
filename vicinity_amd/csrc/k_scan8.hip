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
    uint64_t* keys;  // (distance key << 32) | insertion index
    uint32_t* pos;   // list-major position of the entry
    uint16_t* probe; // probe slot (which probed list)
    uint32_t* count;
    uint32_t* thr;   // distance key threshold: accept fkey(dist) <= thr
};

// Sort the buffer and keep the best `keep` entries; later candidates must beat
// the keep-th distance.  All threads call it.
__device__ void topk_flush(TopkLds& t, int keep) {
    __syncthreads();
    int n = (int)*t.count;
    int n2 = next_pow2(n > 0 ? n : 1);
    for (int i = n + threadIdx.x; i < n2; i += blockDim.x) {
        t.keys[i] = ~0ull;
        t.pos[i] = 0;
        t.probe[i] = 0;
    }
    block_bitonic_sort2(t.keys, t.pos, t.probe, n2);
    if (threadIdx.x == 0) {
        if (n >= keep) {
            *t.thr = (uint32_t)(t.keys[keep - 1] >> 32);
            *t.count = (uint32_t)keep;
        }
    }
    __syncthreads();
}

__device__ __forceinline__ void topk_push(TopkLds& t, bool take, uint32_t fk, uint32_t pos,
                                          int probe, const uint32_t* __restrict__ list_ids) {
    int slot = wave_append_slot(take, t.count);
    if (take) {
        uint32_t vidx = list_ids[pos];
        t.keys[slot] = ((uint64_t)fk << 32) | vidx;
        t.pos[slot] = pos;
        t.probe[slot] = (uint16_t)probe;
    }
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
    uint32_t* lbeg; // [P]
    uint32_t* llen; // [P]
    uint32_t* lid;  // [P]
    uint32_t* pref; // [P+1]
    float* term0;   // [P]
    TopkLds tk;
    uint32_t* misc; // [4 + 2 SCAN_WAVES]
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

__host__ __device__ inline size_t scan_lds_layout(int d, int M, int K, int P, int buf,
                                                  size_t* off /* 12 */) {
    size_t o = 0;
    off[0] = o; o = align16(o + (size_t)d * 4);          // qs
    off[1] = o; o = align16(o + (size_t)d * 4);          // rsd
    off[2] = o; o = align16(o + (size_t)M * K * 4);      // lut
    off[3] = o; o = align16(o + (size_t)P * 4);          // lbeg
    off[4] = o; o = align16(o + (size_t)P * 4);          // llen
    off[5] = o; o = align16(o + (size_t)P * 4);          // lid
    off[6] = o; o = align16(o + (size_t)(P + 1) * 4);    // pref
    off[7] = o; o = align16(o + (size_t)P * 4);          // term0
    off[8] = o; o = align16(o + (size_t)buf * 8);        // keys
    off[9] = o; o = align16(o + (size_t)buf * 4);        // pos
    off[10] = o; o = align16(o + (size_t)buf * 2);       // probe
    off[11] = o; o = align16(o + 4 * (4 + 2 * SCAN_WAVES)); // misc: count, thr, 2 x 8 round counts
    return o;
}

__device__ inline ScanLds carve(char* smem, int d, int M, int K, int P, int buf) {
    size_t off[12];
    scan_lds_layout(d, M, K, P, buf, off);
    ScanLds s;
    s.qs = (float*)(smem + off[0]);
    s.rsd = (float*)(smem + off[1]);
    s.lut = (float*)(smem + off[2]);
    s.lbeg = (uint32_t*)(smem + off[3]);
    s.llen = (uint32_t*)(smem + off[4]);
    s.lid = (uint32_t*)(smem + off[5]);
    s.pref = (uint32_t*)(smem + off[6]);
    s.term0 = (float*)(smem + off[7]);
    s.tk.keys = (uint64_t*)(smem + off[8]);
    s.tk.pos = (uint32_t*)(smem + off[9]);
    s.tk.probe = (uint16_t*)(smem + off[10]);
    s.misc = (uint32_t*)(smem + off[11]);
    s.tk.count = s.misc;
    s.tk.thr = s.misc + 1;
    return s;
}

// Common prologue: query vector and probed list ranges into LDS (the ranges
// only for at most SCAN_LDS_P probes: wider probes are read per slot).
__device__ inline void load_query_and_lists(const DevIndex& ix, const ScanArgs& a, ScanLds& s,
                                            int q) {
    const int tid = threadIdx.x, d = ix.d, P = a.P > SCAN_LDS_P ? 0 : a.P;
    for (int j = tid; j < d; j += blockDim.x) s.qs[j] = a.qn[(size_t)q * d + j];
    for (int p = tid; p < P; p += blockDim.x) {
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
    for (int j = threadIdx.x; j < a.kout; j += blockDim.x) scan_emit(a, q, j, s.tk.keys[j], j < n);
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
        for (int j = tid; j < d; j += blockDim.x) rsd[j] = rr[j];
    } else {
        const float* c = ix.centroids + (size_t)l * d;
        for (int j = tid; j < d; j += blockDim.x) rsd[j] = s.qs[j] - c[j];
    }
}

template <int MT, int KT, int CWD>
__device__ inline void build_table(const DevIndex& ix, const float* rsd, float* lut,
                                   const float (&cw)[cw_count<MT, CWD>()]) {
    const int tid = threadIdx.x;
    const int M = MT > 0 ? MT : ix.M, K = KT > 0 ? KT : ix.K, ds = ix.ds;
    const int t = tid & 255, h = tid >> 8;  // codeword, codebook parity (wave-uniform)
    if constexpr (CWD < 0) {  // ds == W: codewords in registers, the next slice read ahead
        constexpr int W = -CWD;
        float rc[W], rn[W];
#pragma unroll
        for (int j = 0; j < W; j++) rc[j] = h < MT ? rsd[h * W + j] : 0.0f;
#pragma unroll
        for (int i = 0; i < (MT + 1) / 2; i++) {
            const int m = 2 * i + h;
            if (i + 1 < (MT + 1) / 2) {
#pragma unroll
                for (int j = 0; j < W; j++) rn[j] = m + 2 < MT ? rsd[(m + 2) * W + j] : 0.0f;
            }
            float acc = 0.0f;
#pragma unroll
            for (int j = 0; j < W; j++) {
                float diff = rc[j] - cw[i * W + j];
                acc += diff * diff;
            }
            if (m < MT) lut[m * 256 + t] = acc;
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
        for (int e = tid; e < M * K; e += blockDim.x) {
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

// The entries of one list against its table; a block barrier ends every
// round.  The flush decision uses the count every thread holds in tc, so it
// is the same in every wave.
template <int MT, int KT, bool FILT>
__device__ inline void scan_entries(const DevIndex& ix, const ScanArgs& a, ScanLds& s, int buf, const float* lut,
                                    uint32_t beg, uint32_t len, int p, const uint8_t* __restrict__ ecat,
                                    uint8_t cq, TopkCnt& tc) {
    const int tid = threadIdx.x;
    const int M = MT > 0 ? MT : ix.M, K = KT > 0 ? KT : ix.K;
    for (uint32_t base = 0; base < len; base += SCAN_ROUND) {
        if (tc.n > (uint32_t)(buf - SCAN_ROUND)) {
            topk_flush(s.tk, a.kk);
            tc.n = tc.n >= (uint32_t)a.kk ? (uint32_t)a.kk : tc.n;  // the flush keeps kk when it has them
        }
        const uint32_t thr = *s.tk.thr;
        uint32_t wn = 0;  // this wave's appends in the round
#pragma unroll
        for (int u = 0; u < SCAN_U; u++) {
            uint32_t i = base + u * SCAN_THREADS + tid;
            bool take = false;
            uint32_t fk = 0, pos = 0;
            if (i < len) {
                pos = beg + i;
                if (!FILT || ecat[pos] == cq) {
                    float dist = adc_sum<MT, KT>(ix.codes + (size_t)pos * M, lut, M, K, 0.0f);
                    fk = fkey(dist);
                    take = fk <= thr;
                }
            }
            wn += (uint32_t)__popcll(__ballot(take));
            topk_push(s.tk, take, fk, pos, p, ix.list_ids);
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
    scan_entries<MT, KT, FILT>(ix, a, s, buf, s.lut, beg, len, p, ecat, cq, tc);
}

// Codeword t = tid % 256 of the codebooks h, h + 2, ... (h = tid / 256) into
// registers (ksub 256): CWD > 0 holds ds <= CWD floats per codeword, CWD < 0
// exactly ds = -CWD.  The per-list tables then read no codebook memory.
template <int MT, int CWD>
__device__ inline void load_codewords(const DevIndex& ix, float (&cw)[cw_count<MT, CWD>()]) {
    if constexpr (CWD != 0) {
        constexpr int W = CWD > 0 ? CWD : -CWD;
        const int t = threadIdx.x & 255, h = threadIdx.x >> 8, ds = CWD > 0 ? ix.ds : W;
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
__device__ void exact_query(const DevIndex& ix, const ScanArgs& a, int buf, char* smem, int q) {
    const int tid = threadIdx.x;
    const int d = ix.d, M = MT > 0 ? MT : ix.M, K = KT > 0 ? KT : ix.K, P = a.P;
    const bool wide = P > SCAN_LDS_P;
    ScanLds s = carve(smem, d, M, K, wide ? 0 : P, buf);
    float cw[cw_count<MT, CWD>()];
    load_codewords<MT, CWD>(ix, cw);
    load_query_and_lists(ix, a, s, q);
    // list, begin and length of probe slot p (the same for every thread)
    auto slot = [&](int p, uint32_t& l, uint32_t& beg, uint32_t& len) {
        if (wide) {
            l = a.probe[(size_t)q * P + p];
            const bool ok = l < (uint32_t)ix.L;
            beg = ok ? ix.offsets[l] : 0u;
            len = ok ? ix.offsets[l + 1] - beg : 0u;
        } else {
            l = s.lid[p];
            beg = s.lbeg[p];
            len = s.llen[p];
        }
    };
    uint32_t total = 0;
    TopkCnt tc;
    for (int p = 0; p < P; p++) {
        __syncthreads();
        uint32_t l, beg, len;
        slot(p, l, beg, len);
        total += len;
        if (len == 0) continue;
        scan_list<MT, KT, false, CWD>(ix, a, s, buf, l, beg, len, q, p, nullptr, 0, cw, tc);
    }
    topk_flush(s.tk, a.kk);
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
    for (int j = tid; j < d; j += blockDim.x) s.qs[j] = a.qn[(size_t)q * d + j];
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
    topk_flush(s.tk, a.kk);
    const int n = (int)*s.tk.count;
    write_out(a, s, q, n < a.kout ? n : a.kout);
}

template <int MT, int KT, int CWD>
__global__ __launch_bounds__(SCAN_THREADS, 4) void scan8_exact_kernel(DevIndex ix, ScanArgs a, int buf) {
    extern __shared__ __align__(16) char smem[];
    // Every query of the batch (block q takes query q), or the flagged queries
    // the FAST kernel listed before this launch (blocks stride over the list).
    // One call site, so the query body is inlined once.
    const uint32_t nf = a.only_flagged ? *a.flag_count : (uint32_t)a.nq;
    const uint32_t step = a.only_flagged ? gridDim.x : nf;
    for (uint32_t fi = blockIdx.x; fi < nf; fi += step) {
        __syncthreads();
        const int q = a.only_flagged ? (int)a.flag_list[fi] : (int)fi;
        exact_query<MT, KT, CWD>(ix, a, buf, smem, q);
    }
}

// Codewords held per thread: ksub 256 with a fixed codebook count and
// d <= 128 (M * ds floats per thread); 0 = read the codebooks per list.  The
// kernels take -cw_regs when ds is exactly that width.
template <int MT, int KT>
constexpr int cw_regs() {
    return (KT == 256 && MT > 0 && MT <= 64) ? 128 / MT : 0;
}

size_t scan8_lds_bytes(const DevIndex& ix, const ScanArgs& a) {
    size_t off[12];
    return scan_lds_layout(ix.d, ix.M, ix.K, a.P > SCAN_LDS_P ? 0 : a.P, scan_buf(a.kk), off);
}

template <int MT, int KT>
static void launch_mk(const DevIndex& ix, const ScanArgs& a, hipStream_t s) {
    int buf = scan_buf(a.kk);
    size_t lds = scan8_lds_bytes(ix, a);
    constexpr int CWD = cw_regs<MT, KT>();
    auto k = (CWD > 0 && ix.ds == CWD)  ? scan8_exact_kernel<MT, KT, -CWD>
             : (CWD > 0 && ix.ds < CWD) ? scan8_exact_kernel<MT, KT, CWD>
                                        : scan8_exact_kernel<MT, KT, 0>;
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
    size_t off[12];
    const size_t lds = scan_lds_layout(ix.d, ix.M, ix.K, 0, buf, off);
    constexpr int CWD = cw_regs<MT, KT>();
    auto k = (CWD > 0 && ix.ds == CWD)  ? scan8_filtered_kernel<MT, KT, -CWD>
             : (CWD > 0 && ix.ds < CWD) ? scan8_filtered_kernel<MT, KT, CWD>
                                        : scan8_filtered_kernel<MT, KT, 0>;
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
