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
//   coarse_topp_kernel   one wave per query: rescores the candidates with the
//       reference's sequential dot (cosine_distance_normalized,
//       src/distance.rs:104-109), sorts by (score, list) and writes the P
//       smallest in order (find_nearest_centroids, search.rs:1602-1617).  A
//       query whose candidate set may be incomplete goes to
//       launch_coarse_exact_flagged.
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

// Dynamic LDS of the fused kernel, in turn: the normalisation tile
// [FC_QB][d + 1] floats; two pipeline stages of (hi, lo) centroid chunks; the
// waves' key lists [FC_QBW][FC_NH][4][J][64]; then [FC_QB] norms and bounds.
__host__ __device__ inline size_t fc_stage_chunks(int DT) { return (size_t)FC_ST * DT * 4 * 16; }
__host__ __device__ inline size_t fc_main_bytes(int d, int DT, int J) {
    const size_t tile = (size_t)FC_QB * (d + 1) * 4;
    const size_t stages = 2 * 2 * fc_stage_chunks(DT) * 16;
    const size_t merge = (size_t)FC_QBW * FC_NH * 4 * J * 64 * 4;
    size_t m = tile > stages ? tile : stages;
    return m > merge ? m : merge;
}
__host__ __device__ inline size_t fc_lds_bytes(int d, int DT, int J) {
    return fc_main_bytes(d, DT, J) + FC_QB * 2 * 4;
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
template <int DT, int J>
__global__ __launch_bounds__(FC_THREADS) void coarse_fused_kernel(
    const float* __restrict__ Q, int nq, int d, const uint4* __restrict__ Cb, int L, float cmax,
    int Pe, int IB, int normalize, float* __restrict__ qn_out, float* __restrict__ qnorm_out,
    uint32_t* __restrict__ cand, uint32_t* __restrict__ cand_n, uint32_t* __restrict__ qbad,
    unsigned int* __restrict__ nbad) {
    extern __shared__ __align__(16) char smem[];
    constexpr int CAP = 32 * J;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, g = lane >> 4, c = lane & 15;
    const int qb = wave % FC_QBW;
    const int h = __builtin_amdgcn_readfirstlane(wave / FC_QBW);
    const int q0 = blockIdx.x * FC_QB;
    const int rows = min(FC_QB, nq - q0);
    float* tile = reinterpret_cast<float*>(smem);
    float* snorm = reinterpret_cast<float*>(smem + fc_main_bytes(d, DT, J));  // [FC_QB] norm, [FC_QB] bound
    const int st = d + 1;

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
    __syncthreads();  // the tile region becomes the pipeline buffers

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
#pragma unroll
    for (int rr = 0; rr < FC_RPW; rr++) {
        const int r = FC_RPW * h + rr;
        const int row = qb * 16 + 4 * g + r;
        float lst[FC_NH][J];  // the FC_NH waves' lists of this (lane, row)
#pragma unroll
        for (int w = 0; w < FC_NH; w++)
#pragma unroll
            for (int j = 0; j < J; j++) lst[w][j] = mg[((((qb * FC_NH + w) * 4 + r) * J + j) << 6) + lane];
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
        if (row < rows) {
            uint32_t* out = cand + (size_t)(q0 + row) * CAP + (incl - n);
            if (!any_over) {
                uint32_t o = 0;
#pragma unroll
                for (int w = 0; w < FC_NH; w++) {
#pragma unroll
                    for (int j = 0; j < J; j++)
                        if ((uint32_t)j < nw[w]) out[o + j] = 16u * (__float_as_uint(lst[w][j]) & ~kmask) + (uint32_t)c;
                    o += nw[w];
                }
            }
            if (c == 0) cand_n[q0 + row] = any_over ? (uint32_t)CAP + 1u : total;
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
static void launch_fused(const float* Q, int nq, int d, const uint4* Cb, int L, float cmax, int Pe,
                         int normalize, float* qn, float* qnorm, uint32_t* cand, uint32_t* cand_n,
                         hipStream_t s, uint32_t* qbad, unsigned int* nbad) {
    const size_t lds = fc_lds_bytes(d, DT, J);
    // index bits: tiles ceil(L / 16) <= 2^IB
    int IB = 0;
    while ((1 << IB) < (L + 15) / 16) IB++;
    auto k = coarse_fused_kernel<DT, J>;
    ensure_dyn_lds((const void*)k, lds);
    hipLaunchKernelGGL(k, dim3((nq + FC_QB - 1) / FC_QB), dim3(FC_THREADS), lds, s, Q, nq, d, Cb, L, cmax,
                       Pe, IB, normalize, qn, qnorm, cand, cand_n, qbad, nbad);
}

template <int DT>
static void launch_fused_j(const float* Q, int nq, int d, const uint4* Cb, int L, float cmax, int Pe,
                           int normalize, float* qn, float* qnorm, uint32_t* cand, uint32_t* cand_n,
                           hipStream_t s, uint32_t* qbad, unsigned int* nbad) {
    if (fc_keys(Pe) == FC_J_WIDE)
        launch_fused<DT, FC_J_WIDE>(Q, nq, d, Cb, L, cmax, Pe, normalize, qn, qnorm, cand, cand_n, s, qbad, nbad);
    else
        launch_fused<DT, FC_J>(Q, nq, d, Cb, L, cmax, Pe, normalize, qn, qnorm, cand, cand_n, s, qbad, nbad);
}

void launch_coarse_fused(const float* Q, int nq, int d, const uint4* Cb, int L, float cmax, int P,
                         int normalize, float* qn, float* qnorm, uint32_t* cand, uint32_t* cand_n,
                         hipStream_t s, uint32_t* qbad, unsigned int* nbad) {
    if (nq <= 0) return;
    const int Pe = P < L ? P : L;
    switch ((d + 31) / 32) {
        case 1: launch_fused_j<1>(Q, nq, d, Cb, L, cmax, Pe, normalize, qn, qnorm, cand, cand_n, s, qbad, nbad); break;
        case 2: launch_fused_j<2>(Q, nq, d, Cb, L, cmax, Pe, normalize, qn, qnorm, cand, cand_n, s, qbad, nbad); break;
        case 3: launch_fused_j<3>(Q, nq, d, Cb, L, cmax, Pe, normalize, qn, qnorm, cand, cand_n, s, qbad, nbad); break;
        default: launch_fused_j<4>(Q, nq, d, Cb, L, cmax, Pe, normalize, qn, qnorm, cand, cand_n, s, qbad, nbad); break;
    }
}

// ---- exact ordering of the candidates, one wave per query ---------------
#define TP_QD 512

// E: keys per lane, candidate rows of up to 64 E.
template <int E>
__global__ __launch_bounds__(256) void coarse_topp_kernel(
    const uint32_t* __restrict__ cand, const uint32_t* __restrict__ cand_n, int CAP,
    const float* __restrict__ qn, const float* __restrict__ C, int nq, int L, int d, int P,
    uint32_t* __restrict__ probe, uint32_t* __restrict__ flag_list, uint32_t* flag_count) {
    __shared__ float wq[4][TP_QD];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int q = blockIdx.x * 4 + wave;
    if (q >= nq) return;  // per wave: no block barriers below
    const int Pe = P < L ? P : L;
    const uint32_t n = cand_n[q];
    if (n > (uint32_t)CAP) {
        if (lane == 0) flag_list[atomicAdd(flag_count, 1u)] = (uint32_t)q;
        return;
    }
    float* qs = wq[wave];
    for (int j = lane; j < d; j += 64) qs[j] = qn[(size_t)q * d + j];
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
    __builtin_amdgcn_wave_barrier();
    uint64_t kv[E];
#pragma unroll
    for (int e = 0; e < E; e++) {
        const uint32_t t = e * 64 + lane;
        kv[e] = ~0ull;
        if (t < n) {
            const uint32_t cidx = cand[(size_t)q * CAP + t];
            kv[e] = cand_key(1.0f - seq_dot_stream(qs, C + (size_t)cidx * d, d), cidx);
        }
    }
    if (n <= 64) {
        uint64_t k1[1] = {kv[0]};
        wave_sort_regs<1>(k1);
        if (lane < Pe) probe[(size_t)q * P + lane] = (uint32_t)k1[0];
    } else if (n <= 128) {
        uint64_t k2[2] = {kv[0], kv[1]};
        wave_sort_regs<2>(k2);
#pragma unroll
        for (int e = 0; e < 2; e++)
            if (e * 64 + lane < Pe) probe[(size_t)q * P + e * 64 + lane] = (uint32_t)k2[e];
    } else if (E == 4 || n <= 256) {
        uint64_t k4[4] = {kv[0], kv[1], kv[2], kv[3]};
        wave_sort_regs<4>(k4);
#pragma unroll
        for (int e = 0; e < 4; e++)
            if (e * 64 + lane < Pe) probe[(size_t)q * P + e * 64 + lane] = (uint32_t)k4[e];
    } else {
        wave_sort_regs<E>(kv);
#pragma unroll
        for (int e = 0; e < E; e++)
            if (e * 64 + lane < Pe) probe[(size_t)q * P + e * 64 + lane] = (uint32_t)kv[e];
    }
}

void launch_coarse_topp(const uint32_t* cand, const uint32_t* cand_n, int P, const float* qn,
                        const float* C, int nq, int L, int d, uint32_t* probe, uint32_t* flag_list,
                        uint32_t* flag_count, hipStream_t s) {
    if (nq <= 0) return;
    const int Pe = P < L ? P : L;
    const int cap = coarse_fused_cap(Pe);
    static_assert(32 * FC_J <= 256 && 32 * FC_J_WIDE <= 512, "keys per lane");
    if (cap <= 256)
        hipLaunchKernelGGL(coarse_topp_kernel<4>, dim3((nq + 3) / 4), dim3(VGPU_BLOCK), 0, s, cand, cand_n, cap,
                           qn, C, nq, L, d, P, probe, flag_list, flag_count);
    else
        hipLaunchKernelGGL(coarse_topp_kernel<8>, dim3((nq + 3) / 4), dim3(VGPU_BLOCK), 0, s, cand, cand_n, cap,
                           qn, C, nq, L, d, P, probe, flag_list, flag_count);
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
