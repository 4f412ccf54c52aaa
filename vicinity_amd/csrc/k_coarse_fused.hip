// Coarse quantiser in two kernels, without a query x centroid score matrix:
//
//   coarse_fused_kernel  48 queries per workgroup.  Normalises its queries
//       (search.rs:55-62, writes qn), then makes one pass of bf16x3 MFMA dot
//       products against every centroid: q.c ~ qh.ch + qh.cl + ql.ch with
//       x = xh + xl + O(2^-16 |x|) split into bfloat16 halves.  Each (lane, query)
//       keeps the J largest products of the lane's column class, packed with
//       their list index into one float key; two waves share a query block and
//       merge their lists.  The keys above a threshold derived from the P-th
//       largest key and the error bounds are the query's candidates.
//       At its end each wave takes four of the workgroup's queries in turn:
//       it rescores their candidates with the reference's sequential dot
//       (cosine_distance_normalized, src/distance.rs:104-109), sorts them by
//       (score, list) and writes the P smallest in order
//       (find_nearest_centroids, search.rs:1602-1617).  A query whose
//       candidate set may be incomplete goes to launch_coarse_exact_flagged.
//
// MFMA layout (v_mfma_f32_16x16x32_bf16, wave64): lane l holds row/column
// l % 16 and eight consecutive k of group l / 16 for A and B; the result
// element (4 (l / 16) + i, l % 16) sits in element i of lane l.  A and B use
// the same dimension-to-(group, slot) assignment, so every dimension is
// summed exactly once.
#include "vgpu_device.h"
#include "vgpu_bounds.h"
#include "vgpu_launch.h"

namespace vgpu {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float floatx4 __attribute__((ext_vector_type(4)));
// Native 128-bit vector (HIP's uint4 is a struct whose copies stay in memory).
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

#define FC_QBW 3               // query blocks (16 queries each) per workgroup
#define FC_QB (16 * FC_QBW)    // queries per workgroup
#define FC_NH 4                // waves per query block; each takes its own tiles of a stage
#define FC_SUB 1               // 16-centroid tiles per wave and stage
#define FC_ST (FC_NH * FC_SUB) // tiles per stage
#define FC_TR 4                // keys per list that enter the rank (<= FC_J)
#define FC_THREADS (FC_QBW * FC_NH * 64)  // threads per workgroup
#define FC_RPW (4 / FC_NH)     // rows of a lane's four that each wave finishes
static_assert(4 % FC_NH == 0, "wave roles");

// Round to nearest even bfloat16 (finite inputs).
__device__ __forceinline__ uint32_t bf16_bits(float x) {
    const uint32_t u = __float_as_uint(x);
    return (u + 0x7fffu + ((u >> 16) & 1u)) >> 16;
}

// x = hi + lo + r with |r| <= 2^-16 |x| (each rounding to bfloat16 is within
// 2^-8 relative); returns (hi, lo) bit patterns.
__device__ __forceinline__ void bf16_split(float x, uint32_t& hi, uint32_t& lo) {
    hi = bf16_bits(x);
    const float rem = x - __uint_as_float(hi << 16);  // exact (Sterbenz)
    lo = bf16_bits(rem);
}

// Pack centroids into bf16 hi/lo chunks in the order the MFMA tiles read them
// from LDS, so a pipeline stage is one contiguous copy: chunk
// Cb[(((tile * 2 + h) * DT + t) * 4 + g) * 16 + c % 16], tile = c / 16, holds
// the eight dimensions 32 t + 8 g .. + 7 of centroid c (h = 0: hi, 1: lo),
// zero beyond d and for the padding centroids L .. Lp - 1 (Lp = L rounded up
// to a whole pipeline stage, so stage loads need no bounds).
__global__ void coarse_bf16_pack_kernel(const float* __restrict__ C, int L, int Lp, int d, int DT,
                                        uint4* __restrict__ Cb) {
    const size_t e = (size_t)blockIdx.x * blockDim.x + threadIdx.x;  // (c, t, g)
    if (e >= (size_t)Lp * DT * 4) return;
    const int g = (int)(e & 3), t = (int)((e >> 2) % DT);
    const size_t c = e / ((size_t)DT * 4);
    uint32_t h[8], l[8];
#pragma unroll
    for (int i = 0; i < 8; i++) {
        const int j = 32 * t + 8 * g + i;
        bf16_split(j < d && c < (size_t)L ? C[c * d + j] : 0.0f, h[i], l[i]);
    }
    const size_t hi = (((c >> 4) * 2 * DT + t) * 4 + g) * 16 + (c & 15);
    Cb[hi] = make_uint4(h[0] | h[1] << 16, h[2] | h[3] << 16, h[4] | h[5] << 16, h[6] | h[7] << 16);
    Cb[hi + (size_t)DT * 64] =
        make_uint4(l[0] | l[1] << 16, l[2] | l[3] << 16, l[4] | l[5] << 16, l[6] | l[7] << 16);
}

static int fc_padded_lists(int L) { return (L + FC_ST * 16 - 1) / (FC_ST * 16) * (FC_ST * 16); }

size_t coarse_bf16_pack_chunks(int L, int d) { return (size_t)fc_padded_lists(L) * ((d + 31) / 32) * 8; }

void launch_coarse_bf16_pack(const float* C, int L, int d, uint4* Cb, hipStream_t s) {
    const int DT = (d + 31) / 32, Lp = fc_padded_lists(L);
    const size_t n = (size_t)Lp * DT * 4;
    if (n == 0) return;
    hipLaunchKernelGGL(coarse_bf16_pack_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, C,
                       L, Lp, d, DT, Cb);
}

// Dynamic LDS of the fused kernel: one region used in turn by two pipeline
// stages of (hi, lo) centroid chunks, the waves' key lists
// [FC_QBW][FC_NH][4][J][64] and the candidate rows [FC_QB][32 J] with their
// keys, later exact scores; then the query tile [FC_QB][fc_tile_stride(d)]
// floats (kept for the exact rescoring); then [FC_QB] norms, bounds,
// candidate counts, score margins and counts of candidates to rescore.
__host__ __device__ inline size_t fc_stage_chunks(int DT) { return (size_t)FC_ST * DT * 4 * 16; }
__host__ __device__ inline size_t fc_main_bytes(int DT, int J) {
    const size_t stages = 2 * 2 * fc_stage_chunks(DT) * 16;
    const size_t merge = (size_t)FC_QBW * FC_NH * 4 * J * 64 * 4;
    const size_t rows = 2 * (size_t)FC_QB * 32 * J * 4;  // candidate lists and their scores
    size_t m = stages > merge ? stages : merge;
    return m > rows ? m : rows;
}
// query tile row stride: a multiple of four floats (16-byte aligned rows)
__host__ __device__ inline int fc_tile_stride(int d) { return (d & ~3) + 4; }
__host__ __device__ inline size_t fc_tile_bytes(int d) { return (size_t)FC_QB * fc_tile_stride(d) * 4; }
__host__ __device__ inline size_t fc_lds_bytes(int d, int DT, int J) {
    return fc_main_bytes(DT, J) + fc_tile_bytes(d) + FC_QB * 5 * 4;
}

// One pass over all centroids.  The wave with role (qb, h) = (wave % FC_QBW,
// wave / FC_QBW) computes, for tiles h * FC_SUB .. + FC_SUB - 1 of every stage
// of FC_ST 16-centroid tiles, acc = Q_qb . C_tile^T (16 x 16, bf16x3) and hands
// it to `epi(acc, col_base, masked)`, col_base the tile's first centroid and
// masked = the tile may reach past L (only in the last stage).  Stages are
// double-buffered in LDS with one barrier each and loaded two stages ahead
// into registers; a stage's epilogue runs after the next stage's MFMAs are
// issued, so the two overlap.  All threads call this.
template <int DT, typename Epi>
__device__ __forceinline__ void fc_pass(const uint4* __restrict__ Cb_in, int L, const u32x4 (&ah)[DT],
                                        const u32x4 (&al)[DT], u32x4* lds, Epi epi) {
    const u32x4* Cb = reinterpret_cast<const u32x4*>(Cb_in);
    constexpr int SC = FC_ST * DT * 4 * 16;  // chunks per stage and half
    // chunks each thread copies per stage; with 768 threads the last slot is
    // only partly used, so a thread copies slot i only when it exists
    constexpr int PER = (2 * SC + FC_THREADS - 1) / FC_THREADS;
    constexpr bool EXACT_SPLIT = (2 * SC) % FC_THREADS == 0;
    const int tid = threadIdx.x, lane = tid & 63, g = lane >> 4, c = lane & 15;
    const int h = __builtin_amdgcn_readfirstlane((tid >> 6) / FC_QBW);
    const int nst = (L + FC_ST * 16 - 1) / (FC_ST * 16);
    // A stage is 2 SC contiguous chunks of Cb (padded to whole stages), copied
    // to LDS unchanged: slot i of thread tid is chunk i * FC_THREADS + tid.
    // Buffer loads: per-lane offset in a VGPR, stage and slot offsets in
    // SGPRs.  Only stages below nst are fetched.
    const __amdgpu_buffer_rsrc_t rsrc = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<u32x4*>(Cb), (short)0, nst * 2 * SC * 16, 0x00020000);
    const uint32_t lofs = (uint32_t)tid * 16u;
    // One register set: stage st + 1 is stored from it at the start of stage
    // st and stage st + 2 loads into it, so a stage's loads have one stage
    // to arrive (the other waves of the CU cover the rest).
    u32x4 pa[PER];
#define FC_FETCH(SET, ST)                                                              \
    _Pragma("unroll") for (int i = 0; i < PER; i++) if (EXACT_SPLIT || i * FC_THREADS + tid < 2 * SC) SET[i] = __builtin_amdgcn_raw_buffer_load_b128( \
        rsrc, lofs, (uint32_t)((ST) * 2 * SC * 16 + i * FC_THREADS * 16), 0);
#define FC_STORE(SET, BUF)                                                             \
    _Pragma("unroll") for (int i = 0; i < PER; i++) if (EXACT_SPLIT || i * FC_THREADS + tid < 2 * SC) lds[(size_t)(BUF) * 2 * SC + i * FC_THREADS + tid] = SET[i];
    floatx4 prev[FC_SUB];
    // Stage ST: everyone has finished stage ST - 1 (buffer (ST + 1) & 1) and
    // stage ST's chunks are visible; SET holds stage ST + 1, then ST + 2.
#define FC_STEP(ST, SET)                                                               \
    {                                                                                  \
        const int st_ = (ST);                                                          \
        __syncthreads();                                                               \
        if (st_ + 1 < nst) {                                                           \
            FC_STORE(SET, (st_ + 1) & 1)                                               \
            if (st_ + 2 < nst) { FC_FETCH(SET, st_ + 2) }                              \
        }                                                                              \
        const u32x4* b = lds + (size_t)(st_ & 1) * 2 * SC;                             \
        floatx4 acc[FC_SUB];                                                           \
        _Pragma("unroll") for (int sub = 0; sub < FC_SUB; sub++) acc[sub] = floatx4{0.f, 0.f, 0.f, 0.f}; \
        _Pragma("unroll") for (int t = 0; t < DT; t++) {                               \
            bf16x8 bh[FC_SUB], bl[FC_SUB];                                             \
            _Pragma("unroll") for (int sub = 0; sub < FC_SUB; sub++) {                 \
                const int o = (((h * FC_SUB + sub) * 2 * DT + t) * 4 + g) * 16 + c;    \
                bh[sub] = __builtin_bit_cast(bf16x8, b[o]);                            \
                bl[sub] = __builtin_bit_cast(bf16x8, b[o + DT * 64]);                  \
            }                                                                          \
            const bf16x8 a_h = __builtin_bit_cast(bf16x8, ah[t]);                      \
            const bf16x8 a_l = __builtin_bit_cast(bf16x8, al[t]);                      \
            _Pragma("unroll") for (int sub = 0; sub < FC_SUB; sub++)                   \
                acc[sub] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a_h, bl[sub], acc[sub], 0, 0, 0); \
            _Pragma("unroll") for (int sub = 0; sub < FC_SUB; sub++)                   \
                acc[sub] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a_l, bh[sub], acc[sub], 0, 0, 0); \
            _Pragma("unroll") for (int sub = 0; sub < FC_SUB; sub++)                   \
                acc[sub] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a_h, bh[sub], acc[sub], 0, 0, 0); \
        }                                                                              \
        if (st_ > 0) { /* stage st_ - 1 < nst - 1 is whole */                          \
            _Pragma("unroll") for (int sub = 0; sub < FC_SUB; sub++)                   \
                epi(prev[sub], ((st_ - 1) * FC_ST + h * FC_SUB + sub) * 16, false);    \
        }                                                                              \
        _Pragma("unroll") for (int sub = 0; sub < FC_SUB; sub++) prev[sub] = acc[sub]; \
    }
    FC_FETCH(pa, 0)
    FC_STORE(pa, 0)
    if (nst > 1) { FC_FETCH(pa, 1) }
    for (int st = 0; st < nst; st++) FC_STEP(st, pa)
#undef FC_STEP
    const bool masked = nst * FC_ST * 16 > L;
#pragma unroll
    for (int sub = 0; sub < FC_SUB; sub++) epi(prev[sub], ((nst - 1) * FC_ST + h * FC_SUB + sub) * 16, masked);
#undef FC_FETCH
#undef FC_STORE
}

// bf16 hi/lo A operands of one row, element j = x(j), dimensions
// 32 t + 8 g .. + 7 for lane group g.
template <int DT, typename X>
__device__ __forceinline__ void fc_split_rows(X x, int d, int g, u32x4 (&ah)[DT], u32x4 (&al)[DT]) {
#pragma unroll
    for (int t = 0; t < DT; t++) {
        uint32_t hb[8], lb[8];
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const int j = 32 * t + 8 * g + i;
            bf16_split(j < d ? x(j) : 0.0f, hb[i], lb[i]);
        }
        ah[t] = u32x4{hb[0] | hb[1] << 16, hb[2] | hb[3] << 16, hb[4] | hb[5] << 16, hb[6] | hb[7] << 16};
        al[t] = u32x4{lb[0] | lb[1] << 16, lb[2] | lb[3] << 16, lb[4] | lb[5] << 16, lb[6] | lb[7] << 16};
    }
}

// Rank k (0-based, ascending) among the 16 J keys held by the 16 lanes of
// this lane's 16-lane group, J per lane (bitonic sort over element
// e * 16 + lane % 16; strides below 16 stay inside the group).
template <int J>
__device__ __forceinline__ uint32_t group16_rank(uint32_t (&v)[J], int k) {
    const int l16 = threadIdx.x & 15;
#pragma unroll
    for (int size = 2; size <= 16 * J; size <<= 1) {
#pragma unroll
        for (int stride = size >> 1; stride > 0; stride >>= 1) {
            if (stride >= 16) {
                const int es = stride >> 4;
#pragma unroll
                for (int e = 0; e < J; e++) {
                    const int f = e ^ es;
                    if (f > e) {
                        const bool asc = (((e << 4) | l16) & size) == 0;
                        const uint32_t a = v[e], b = v[f];
                        const bool sw = (a > b) == asc;
                        v[e] = sw ? b : a;
                        v[f] = sw ? a : b;
                    }
                }
            } else {
#pragma unroll
                for (int e = 0; e < J; e++) {
                    const uint32_t o = shfl_xor_u32(v[e], stride);
                    const bool asc = (((e << 4) | l16) & size) == 0;
                    const bool lower = (l16 & stride) == 0;
                    v[e] = (lower == asc) ? (o < v[e] ? o : v[e]) : (o > v[e] ? o : v[e]);
                }
            }
        }
    }
    uint32_t x = v[0];
#pragma unroll
    for (int e = 1; e < J; e++) x = (k >> 4) == e ? v[e] : x;
    return __shfl(x, (threadIdx.x & 48) | (k & 15), 64);
}

// Insert v into the descending list t[0] >= .. >= t[J-1] (the J largest of
// the list and v): t_i' = med3(t_{i-1}, t_i, v), updated from the bottom so
// each step reads the old t_{i-1}; t_0' = max(t_0, v) as med3 against a
// finite bound above every key.
template <int J>
__device__ __forceinline__ void top_insert(float (&t)[J], float v) {
#pragma unroll
    for (int i = J - 1; i > 0; i--) t[i] = __builtin_amdgcn_fmed3f(t[i - 1], t[i], v);
    t[0] = __builtin_amdgcn_fmed3f(t[0], v, 3.0e38f);
}

// One pass of bf16x3 products.  Every (wave, lane, row) keeps the J largest
// keys k = (a + 2) with its low IB mantissa bits replaced by the tile index
// (a = approximate q.c; the lane's column c = lane % 16 completes the list
// index 16 tile + c); the FC_NH waves of a query block see disjoint tiles, so
// a row has FC_NH x 16 sorted lists of J.  T = the Pe-th largest of the row's
// keys bounds the Pe-th largest approximate dot from below (Pe distinct lists
// have keys >= T, so approximate dots >= T - 2 - E, E the packing error).  Pe
// lists then have exact scores within eps of those, so every list among the
// Pe exact nearest has an approximate dot within 2 eps of T - 2 - E and a key
// >= T - 2E - 2 eps (taken with a factor 1.25 and a few ulps to spare); those
// keys form a prefix of each list.  (T is taken over the lists' first FC_TR
// keys, Pe <= 16 FC_NH FC_TR.)  A list whose J-th key is itself above that
// threshold may have dropped such a list, and a row holds at most CAP
// candidates: the row is then marked overflowed (cand_n = CAP + 1).  After the
// pass wave h finishes rows FC_RPW h .. + FC_RPW - 1 of each lane.  Three
// query blocks of FC_NH waves (48 queries, 12 waves) per workgroup: a 10k
// batch is 209 workgroups, one per CU with none left over (with 32 queries,
// 313 workgroups left 57 CUs running two and the launch waited for them).
// Sequential dots (src/simd.rs:88-91 order, one rounding per product and per
// sum) of G (query, centroid) pairs at once: the centroids stream from global
// memory 32 floats per pair and step, all G pairs' loads in flight together,
// and the G sums interleave.  Rows 16-byte aligned; d % 4 == 0 (else one
// float at a time).
template <int G>
__device__ __forceinline__ void fc_seq_dots(const float* const (&qa)[G], const float* const (&cb)[G], int d,
                                            float (&out)[G]) {
#pragma unroll
    for (int g = 0; g < G; g++) out[g] = 0.0f;
    if (d & 3) {
        for (int j = 0; j < d; j++)
#pragma unroll
            for (int g = 0; g < G; g++) out[g] = __fadd_rn(out[g], __fmul_rn(qa[g][j], cb[g][j]));
        return;
    }
    int j0 = 0;
    for (; j0 + 32 <= d; j0 += 32) {
        float4 v[G][8];
#pragma unroll
        for (int g = 0; g < G; g++)
#pragma unroll
            for (int i = 0; i < 8; i++) v[g][i] = reinterpret_cast<const float4*>(cb[g] + j0)[i];
#pragma unroll
        for (int i = 0; i < 8; i++) {
            float4 a[G];
#pragma unroll
            for (int g = 0; g < G; g++) a[g] = reinterpret_cast<const float4*>(qa[g] + j0)[i];
#pragma unroll
            for (int g = 0; g < G; g++) {
                out[g] = __fadd_rn(out[g], __fmul_rn(a[g].x, v[g][i].x));
                out[g] = __fadd_rn(out[g], __fmul_rn(a[g].y, v[g][i].y));
                out[g] = __fadd_rn(out[g], __fmul_rn(a[g].z, v[g][i].z));
                out[g] = __fadd_rn(out[g], __fmul_rn(a[g].w, v[g][i].w));
            }
        }
    }
    for (; j0 < d; j0 += 4) {
        float4 v[G], a[G];
#pragma unroll
        for (int g = 0; g < G; g++) {
            v[g] = reinterpret_cast<const float4*>(cb[g] + j0)[0];
            a[g] = reinterpret_cast<const float4*>(qa[g] + j0)[0];
        }
#pragma unroll
        for (int g = 0; g < G; g++) {
            out[g] = __fadd_rn(out[g], __fmul_rn(a[g].x, v[g].x));
            out[g] = __fadd_rn(out[g], __fmul_rn(a[g].y, v[g].y));
            out[g] = __fadd_rn(out[g], __fmul_rn(a[g].z, v[g].z));
            out[g] = __fadd_rn(out[g], __fmul_rn(a[g].w, v[g].w));
        }
    }
}

// The exact selection of one query from its scored candidate row (n <= 64 E
// (fkey(1 - dot), list) pairs in LDS), one wave: the wave sorts the keys and
// lanes write the Pe smallest lists in order.
template <int E>
__device__ __forceinline__ void fc_select_row(const uint32_t* cand, const uint32_t* score, uint32_t n, int Pe,
                                              uint32_t* __restrict__ probe_row) {
    const int lane = threadIdx.x & 63;
    uint64_t kv[E];
#pragma unroll
    for (int e = 0; e < E; e++) {
        const uint32_t t = e * 64 + lane;
        kv[e] = t < n ? ((uint64_t)score[t] << 32) | cand[t] : ~0ull;
    }
    wave_sort_regs<E>(kv);
#pragma unroll
    for (int e = 0; e < E; e++)
        if (e * 64 + lane < Pe) probe_row[e * 64 + lane] = (uint32_t)kv[e];
}

template <int DT, int J>
__global__ __launch_bounds__(FC_THREADS) void coarse_fused_kernel(
    const float* __restrict__ Q, int nq, int d, const uint4* __restrict__ Cb, int L, float cmax,
    int Pe, int P, int IB, int normalize, int ordered, float* __restrict__ qn_out, float* __restrict__ qnorm_out,
    const float* __restrict__ C, uint32_t* __restrict__ probe, uint32_t* __restrict__ flag_list,
    uint32_t* __restrict__ flag_count, uint32_t* __restrict__ qbad, unsigned int* __restrict__ nbad) {
    extern __shared__ __align__(16) char smem[];
    constexpr int CAP = 32 * J;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, g = lane >> 4, c = lane & 15;
    const int qb = wave % FC_QBW;
    const int h = __builtin_amdgcn_readfirstlane(wave / FC_QBW);
    const int q0 = blockIdx.x * FC_QB;
    const int rows = min(FC_QB, nq - q0);
    float* tile = reinterpret_cast<float*>(smem + fc_main_bytes(DT, J));
    // [FC_QB] norm, [FC_QB] bound, [FC_QB] candidate count
    float* snorm = reinterpret_cast<float*>(smem + fc_main_bytes(DT, J) + fc_tile_bytes(d));
    uint32_t* scnt = reinterpret_cast<uint32_t*>(snorm + 2 * FC_QB);
    float* smar = snorm + 3 * FC_QB;     // [FC_QB] score margin of the keys
    uint32_t* sunc = scnt + 2 * FC_QB;   // [FC_QB] candidates left to rescore
    const int st = fc_tile_stride(d);

    // ---- normalise (search.rs:55-62): sequential sum of squares per row.
    // A row holding a NaN or an infinity is searched as the zero vector,
    // marked in qbad and counted in *nbad (its result row becomes padding).
    const float* src = Q + (size_t)q0 * d;
    for (int e = tid; e < FC_QB * d; e += FC_THREADS) {
        const int r = e / d;
        tile[r * st + e % d] = r < rows ? src[e] : 0.0f;
    }
    __syncthreads();
    if (tid < FC_QB) {
        float* xr = tile + tid * st;
        if (row_nonfinite(xr, d)) {
            for (int j = 0; j < d; j++) xr[j] = 0.0f;
            if (nbad) atomicAdd(nbad, 1u);
            if (qbad && tid < rows) qbad[q0 + tid] = 1u;
        } else if (qbad && tid < rows) {
            qbad[q0 + tid] = 0u;
        }
        float s = 0.0f;
        for (int j = 0; j < d; j++) s = __fadd_rn(s, __fmul_rn(xr[j], xr[j]));
        const float nrm = sqrtf(s);
        // without normalisation the rows are used as given; the bound is ||x||
        snorm[tid] = normalize ? nrm : 0.0f;
        snorm[FC_QB + tid] = normalize && nrm > 1e-10f ? 1.0001f : nrm * 1.0001f + 1e-30f;
        if (tid < rows && qnorm_out) qnorm_out[q0 + tid] = snorm[FC_QB + tid];
    }
    __syncthreads();
    if (normalize) {
        for (int e = tid; e < FC_QB * d; e += FC_THREADS) {
            const int r = e / d, j = e % d;
            const float nrm = snorm[r];
            const float v = tile[r * st + j];
            const float x = nrm > 1e-10f ? v / nrm : v;
            tile[r * st + j] = x;
            if (r < rows) qn_out[(size_t)(q0 + r) * d + j] = x;
        }
        __syncthreads();
    }
    u32x4 ah[DT], al[DT];
    {
        const float* xr = tile + (qb * 16 + c) * st;
        fc_split_rows<DT>([&](int j) { return xr[j]; }, d, g, ah, al);
    }

    // ---- the pass: J largest packed keys per (lane, row 4 g + r).
    const uint32_t kmask = ~((1u << IB) - 1u);
    float top[4][J];
#pragma unroll
    for (int r = 0; r < 4; r++)
#pragma unroll
        for (int j = 0; j < J; j++) top[r][j] = -3.0e38f;  // below every key
    fc_pass<DT>(Cb, L, ah, al, reinterpret_cast<u32x4*>(smem), [&](const floatx4& acc, int cb, bool masked) {
        const uint32_t ti = (uint32_t)cb >> 4;
        const bool valid = !masked || cb + c < L;
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const float k = __uint_as_float((__float_as_uint(acc[r] + 2.0f) & kmask) | ti);
            top_insert<J>(top[r], valid ? k : -3.0e38f);
        }
    });

    // ---- exchange: every wave's lists to LDS [qb][h][r][j][lane].
    __syncthreads();  // the pipeline buffers become the exchange area
    float* mg = reinterpret_cast<float*>(smem);
#pragma unroll
    for (int r = 0; r < 4; r++)
#pragma unroll
        for (int j = 0; j < J; j++) mg[((((qb * FC_NH + h) * 4 + r) * J + j) << 6) + lane] = top[r][j];
    __syncthreads();

    // ---- rows FC_RPW h .. + FC_RPW - 1: threshold, overflow test and output.
    static_assert(FC_RPW == 1, "one row per lane group and wave");
    {
        const int r = h;
        const int row = qb * 16 + 4 * g + r;
        float lst[FC_NH][J];  // the FC_NH waves' lists of this (lane, row)
#pragma unroll
        for (int w = 0; w < FC_NH; w++)
#pragma unroll
            for (int j = 0; j < J; j++) lst[w][j] = mg[((((qb * FC_NH + w) * 4 + r) * J + j) << 6) + lane];
        __syncthreads();  // every list read: the region becomes the candidate rows
        // T = the Pe-th largest of the lists' first FC_TR keys (a subset, so
        // Pe distinct lists still have keys >= T; T is below the full rank
        // only when a list holds more than FC_TR of the top Pe).
        uint32_t kv[FC_NH * FC_TR];
#pragma unroll
        for (int w = 0; w < FC_NH; w++)
#pragma unroll
            for (int j = 0; j < FC_TR; j++) kv[w * FC_TR + j] = fkey(lst[w][j]);
        const float T = fkey_to_float(group16_rank<FC_NH * FC_TR>(kv, 16 * FC_NH * FC_TR - Pe));
        const float qb_norm = snorm[FC_QB + row];
        const float qc = qb_norm * cmax;
        const float u = 5.9604645e-08f;
        // packing: < 2^IB ulps of a + 2 plus half an ulp of its rounding; every
        // |a + 2| <= qc + 2 < ub (a power of two) has ulp <= ub u
        const float ub = __uint_as_float((__float_as_uint(qc + 2.0f) & 0x7f800000u) + 0x00800000u);
        const float E = ((float)(1u << IB) + 0.5f) * ub * u;
        const float kthr = T - (2.0f * E + 2.5f * coarse_eps_bf16(d, qb_norm, cmax) + 8.0f * ub * u);
        uint32_t nw[FC_NH], n = 0;
        bool over = false;
#pragma unroll
        for (int w = 0; w < FC_NH; w++) {
            nw[w] = 0;
#pragma unroll
            for (int j = 0; j < J; j++) nw[w] += lst[w][j] >= kthr ? 1u : 0u;
            n += nw[w];
            over = over || lst[w][J - 1] >= kthr;
        }
        // exclusive prefix of n over the 16 lanes of the group
        uint32_t incl = n;
#pragma unroll
        for (int o = 1; o < 16; o <<= 1) {
            const uint32_t x = __shfl_up(incl, o, 16);
            if (c >= o) incl += x;
        }
        const uint32_t total = __shfl(incl, (lane & 48) | 15, 64);
        // a list that may have dropped a member, or more candidates than a row holds
        const bool any_over = (__ballot(over) >> (16 * g) & 0xffffull) || total > (uint32_t)CAP;
        // candidate lists [row][CAP] and their keys [row][CAP] beside them
        uint32_t* out = reinterpret_cast<uint32_t*>(smem) + (size_t)row * CAP + (incl - n);
        float* okey = reinterpret_cast<float*>(smem) + (size_t)FC_QB * CAP + (size_t)row * CAP + (incl - n);
        if (!any_over) {
            uint32_t o = 0;
#pragma unroll
            for (int w = 0; w < FC_NH; w++) {
#pragma unroll
                for (int j = 0; j < J; j++)
                    if ((uint32_t)j < nw[w]) {
                        out[o + j] = 16u * (__float_as_uint(lst[w][j]) & ~kmask) + (uint32_t)c;
                        okey[o + j] = lst[w][j];
                    }
                o += nw[w];
            }
        }
        if (c == 0) {
            scnt[row] = any_over ? (uint32_t)CAP + 1u : total;
            // a key is within E of a + 2 and a within eps of the reference's
            // dot: the reference score 1 - dot is within this of 3 - key
            smar[row] = E + 1.25f * coarse_eps_bf16(d, qb_norm, cmax) + 4.0f * ub * u;
        }
    }
    __syncthreads();

    // ---- the selection (find_nearest_centroids, search.rs:1602-1617: the Pe
    // smallest reference scores 1 - dot, ties to the lower list).  Wave w
    // takes rows w, w + 12, ...  A candidate's reference score lies within
    // the row's margin m of 3 - key, so one that at least n - Pe others
    // surely trail is among the Pe, one that Pe others surely lead is not,
    // and only the rest are rescored with the reference's sequential dot
    // against the query as searched (distance.rs:104-109) and ranked by
    // (score, list) for the remaining places.  The sure members are a prefix
    // of the order by 3 - key (any candidate ahead of one trails at least as
    // many), so each is written at its place in that order, and the rescored
    // ones follow in rank order: nearest lists first, which tightens the
    // scan's bound soonest.  With `ordered` every candidate is rescored and
    // the Pe lists are written in rank order.
    {
        constexpr int RPW = FC_QB / (FC_THREADS / 64);  // rows per wave
        uint32_t* lc = reinterpret_cast<uint32_t*>(smem);                    // ids [FC_QB][CAP]
        uint32_t* sc = reinterpret_cast<uint32_t*>(smem) + (size_t)FC_QB * CAP;  // keys, then scores
        uint32_t rn[RPW], rbeg[RPW + 1], rin[RPW];
        rbeg[0] = 0;
#pragma unroll
        for (int i = 0; i < RPW; i++) {
            const int row = wave + i * (FC_THREADS / 64);
            uint32_t n = row < rows ? scnt[row] : 0u;
            if (n > (uint32_t)CAP) {  // may be incomplete: the exact fallback
                if (lane == 0) flag_list[atomicAdd(flag_count, 1u)] = (uint32_t)(q0 + row);
                n = 0;
            }
            uint32_t in = 0, un = n;
            if (!ordered && n > 0) {
                uint32_t* ids = lc + (size_t)row * CAP;
                const float* keys = reinterpret_cast<const float*>(sc) + (size_t)row * CAP;
                const float m2 = 2.0f * smar[row];
                uint32_t* pr = probe + (size_t)(q0 + row) * P;
                un = 0;
                // every lane reads its candidates before any slot is rewritten
                constexpr int EM = (32 * J + 63) / 64;
                uint32_t id[EM], st_[EM], ahead[EM];
                float cs[EM];
#pragma unroll
                for (int e = 0; e < EM; e++) {
                    const uint32_t t = e * 64 + lane;
                    id[e] = t < n ? ids[t] : 0u;
                    cs[e] = t < n ? 3.0f - keys[t] : 0.0f;
                    st_[e] = 0u;
                    ahead[e] = 0u;
                }
#pragma unroll
                for (int e = 0; e < EM; e++) {
                    if ((uint32_t)(e * 64) >= n) break;  // wave-uniform
                    const uint32_t t = e * 64 + lane;
                    uint32_t better = 0, worse = 0, a = 0;
                    for (uint32_t j = 0; j < n; j++) {
                        const float cj = 3.0f - keys[j];
                        better += cj + m2 < cs[e] ? 1u : 0u;
                        worse += cj - m2 > cs[e] ? 1u : 0u;
                        a += cj < cs[e] || (cj == cs[e] && j < t) ? 1u : 0u;
                    }
                    ahead[e] = a;
                    st_[e] = t >= n ? 0u : worse >= n - (uint32_t)Pe ? 1u : better >= (uint32_t)Pe ? 0u : 2u;
                }
#pragma unroll
                for (int e = 0; e < EM; e++) {
                    if ((uint32_t)(e * 64) >= n) break;
                    const uint64_t bi = __ballot(st_[e] == 1u), bu = __ballot(st_[e] == 2u);
                    const uint32_t ou = __builtin_amdgcn_mbcnt_hi((uint32_t)(bu >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)bu, 0u));
                    if (st_[e] == 1u && ahead[e] < (uint32_t)Pe) pr[ahead[e]] = id[e];
                    if (st_[e] == 2u) ids[un + ou] = id[e];
                    in += (uint32_t)__popcll(bi);
                    un += (uint32_t)__popcll(bu);
                }
            }
            rn[i] = in < (uint32_t)Pe ? un : 0u;  // no place left: nothing to rescore
            rin[i] = in;
            rbeg[i + 1] = rbeg[i] + rn[i];
        }
        // the candidates left to rescore, numbered in row order: lane l takes
        // numbers l, l + 64, ..., three at a time
        const uint32_t tot = rbeg[RPW];
        constexpr int G = 3;  // pairs per lane in flight (registers: 32 G floats)
        for (uint32_t b0 = 0; b0 < tot; b0 += 64 * G) {
            const float* qa[G];
            const float* cb[G];
            uint32_t at[G];  // LDS slot of each number (row * CAP + t), or ~0
#pragma unroll
            for (int g = 0; g < G; g++) {
                const uint32_t x = b0 + 64 * g + lane;
                int ri = 0;
#pragma unroll
                for (int i = 1; i < RPW; i++) ri += x >= rbeg[i] ? 1 : 0;
                const int row = wave + ri * (FC_THREADS / 64);
                const bool ok = x < tot;
                at[g] = ok ? (uint32_t)row * CAP + (x - rbeg[ri]) : ~0u;
                qa[g] = tile + (ok ? row : 0) * st;
                cb[g] = C + (size_t)(ok ? lc[at[g]] : 0u) * d;
            }
            float dot[G];
            fc_seq_dots<G>(qa, cb, d, dot);
#pragma unroll
            for (int g = 0; g < G; g++)
                if (at[g] != ~0u) sc[at[g]] = fkey(1.0f - dot[g]);
        }
        __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
        __builtin_amdgcn_wave_barrier();
#pragma unroll
        for (int i = 0; i < RPW; i++) {
            const int row = wave + i * (FC_THREADS / 64);
            const uint32_t n = rn[i];
            if (n == 0) continue;  // nothing left to rank, overflowed or past the batch
            const uint32_t* cr = lc + (size_t)row * CAP;
            const uint32_t* sr = sc + (size_t)row * CAP;
            uint32_t* pr = probe + (size_t)(q0 + row) * P + rin[i];
            const int need = Pe - (int)rin[i];
            if (n <= 64) fc_select_row<1>(cr, sr, n, need, pr);
            else if (n <= 128) fc_select_row<2>(cr, sr, n, need, pr);
            else if (n <= 256) fc_select_row<4>(cr, sr, n, need, pr);
            else fc_select_row<8>(cr, sr, n, need, pr);
        }
    }
}

// Keys per (wave, lane, row): 8 up to 32 probes, 10 above, where a list
// holding more than 8 of the window's lists flags the query more often
// (about 5 queries of a 10k batch at 16,384 lists and 64 probes).
#define FC_J 8
#define FC_J_WIDE 10
static int fc_keys(int P) { return P > 32 ? FC_J_WIDE : FC_J; }

int coarse_fused_cap(int P) { return 32 * fc_keys(P); }

bool coarse_fused_supported(int d, int P) { return d >= 1 && d <= 128 && P >= 1 && P <= 64; }

template <int DT, int J>
static void launch_fused(const float* Q, int nq, int d, const uint4* Cb, int L, float cmax, int Pe, int P,
                         int normalize, int ordered, float* qn, float* qnorm, const float* C, uint32_t* probe,
                         uint32_t* flag_list, uint32_t* flag_count, hipStream_t s, uint32_t* qbad,
                         unsigned int* nbad) {
    const size_t lds = fc_lds_bytes(d, DT, J);
    // index bits: tiles ceil(L / 16) <= 2^IB
    int IB = 0;
    while ((1 << IB) < (L + 15) / 16) IB++;
    auto k = coarse_fused_kernel<DT, J>;
    ensure_dyn_lds((const void*)k, lds);
    hipLaunchKernelGGL(k, dim3((nq + FC_QB - 1) / FC_QB), dim3(FC_THREADS), lds, s, Q, nq, d, Cb, L, cmax,
                       Pe, P, IB, normalize, ordered, qn, qnorm, C, probe, flag_list, flag_count, qbad, nbad);
}

template <int DT>
static void launch_fused_j(const float* Q, int nq, int d, const uint4* Cb, int L, float cmax, int Pe, int P,
                           int normalize, int ordered, float* qn, float* qnorm, const float* C, uint32_t* probe,
                           uint32_t* flag_list, uint32_t* flag_count, hipStream_t s, uint32_t* qbad,
                           unsigned int* nbad) {
    if (fc_keys(Pe) == FC_J_WIDE)
        launch_fused<DT, FC_J_WIDE>(Q, nq, d, Cb, L, cmax, Pe, P, normalize, ordered, qn, qnorm, C, probe, flag_list,
                                    flag_count, s, qbad, nbad);
    else
        launch_fused<DT, FC_J>(Q, nq, d, Cb, L, cmax, Pe, P, normalize, ordered, qn, qnorm, C, probe, flag_list,
                               flag_count, s, qbad, nbad);
}

void launch_coarse_fused(const float* Q, int nq, int d, const uint4* Cb, int L, float cmax, int P,
                         int normalize, int ordered, float* qn, float* qnorm, const float* C, uint32_t* probe,
                         uint32_t* flag_list, uint32_t* flag_count, hipStream_t s, uint32_t* qbad,
                         unsigned int* nbad) {
    if (nq <= 0) return;
    const int Pe = P < L ? P : L;
#define FC_L(DTV) launch_fused_j<DTV>(Q, nq, d, Cb, L, cmax, Pe, P, normalize, ordered, qn, qnorm, C, probe, flag_list, \
                                      flag_count, s, qbad, nbad)
    switch ((d + 31) / 32) {
        case 1: FC_L(1); break;
        case 2: FC_L(2); break;
        case 3: FC_L(3); break;
        default: FC_L(4); break;
    }
#undef FC_L
}

// ---- test entry: the bf16x3 dot products of the fused kernel ------------
// D[q][c] = Q[q] . C[c] through fc_pass (Q already normalised or not).
template <int DT>
__global__ __launch_bounds__(FC_THREADS) void coarse_bf16x3_dots_kernel(const float* __restrict__ Q, int nq,
                                                                 int d, const uint4* __restrict__ Cb,
                                                                 int L, float* __restrict__ D) {
    extern __shared__ __align__(16) char smem[];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, g = lane >> 4, c = lane & 15;
    const int qb = wave % FC_QBW;
    const int q0 = blockIdx.x * FC_QB;
    const int row_a = q0 + qb * 16 + c;
    u32x4 ah[DT], al[DT];
    fc_split_rows<DT>([&](int j) { return row_a < nq ? Q[(size_t)row_a * d + j] : 0.0f; }, d, g, ah, al);
    fc_pass<DT>(Cb, L, ah, al, reinterpret_cast<u32x4*>(smem), [&](const floatx4& acc, int cb, bool) {
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const int row = q0 + qb * 16 + 4 * g + r, col = cb + c;
            if (row < nq && col < L) D[(size_t)row * L + col] = acc[r];
        }
    });
}

void launch_coarse_bf16x3_dots(const float* Q, int nq, int d, const uint4* Cb, int L, float* D,
                               hipStream_t s) {
    if (nq <= 0 || L <= 0) return;
    const int DT = (d + 31) / 32;
    const size_t lds = 2 * 2 * fc_stage_chunks(DT) * 16;
    const dim3 grid((nq + FC_QB - 1) / FC_QB);
    switch (DT) {
        case 1:
            ensure_dyn_lds((const void*)coarse_bf16x3_dots_kernel<1>, lds);
            hipLaunchKernelGGL(coarse_bf16x3_dots_kernel<1>, grid, dim3(FC_THREADS), lds, s, Q, nq, d, Cb, L, D);
            break;
        case 2:
            ensure_dyn_lds((const void*)coarse_bf16x3_dots_kernel<2>, lds);
            hipLaunchKernelGGL(coarse_bf16x3_dots_kernel<2>, grid, dim3(FC_THREADS), lds, s, Q, nq, d, Cb, L, D);
            break;
        case 3:
            ensure_dyn_lds((const void*)coarse_bf16x3_dots_kernel<3>, lds);
            hipLaunchKernelGGL(coarse_bf16x3_dots_kernel<3>, grid, dim3(FC_THREADS), lds, s, Q, nq, d, Cb, L, D);
            break;
        default:
            ensure_dyn_lds((const void*)coarse_bf16x3_dots_kernel<4>, lds);
            hipLaunchKernelGGL(coarse_bf16x3_dots_kernel<4>, grid, dim3(FC_THREADS), lds, s, Q, nq, d, Cb, L, D);
            break;
    }
}

}  // namespace vgpu
