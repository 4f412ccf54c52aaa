// Coarse quantiser without a query x centroid score matrix:
//
//   coarse_fused_kernel  48 queries per workgroup of eight waves.  Normalises
//       its queries (search.rs:55-62, writes qn), then every wave holds all 48
//       queries as bf16 hi/lo MFMA operands and makes one pass of bf16x3 dot
//       products, q.c ~ qh.ch + qh.cl + ql.ch with x = xh + xl + O(2^-16 |x|),
//       over its eighth of the centroid tiles (16 centroids each), loading
//       them straight from L2.  Each (wave, lane column, query) keeps the J
//       largest products of its 1/128 of the lists, packed with their tile
//       number into one float key.  The Pe-th largest of a query's 128 list
//       maxima bounds its Pe-th largest key from below (those are Pe distinct
//       lists), and the keys above that bound less the error margins are the
//       query's candidates.  A candidate whose approximate score is surely
//       among the Pe smallest is written at once, one surely outside is
//       dropped, and the rest are rescored with the reference's sequential
//       dot (cosine_distance_normalized, src/distance.rs:104-109) and ranked
//       by (score, list) for the remaining places (find_nearest_centroids,
//       search.rs:1602-1617).  A query whose candidate set may be incomplete
//       goes to launch_coarse_exact_flagged.
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

#define FC_QBW 3                  // query blocks (16 queries each) per workgroup
#define FC_QB (16 * FC_QBW)       // queries per workgroup
#define FC_NW 8                   // waves per workgroup; wave h takes tiles h, h + FC_NW, ...
#define FC_THREADS (FC_NW * 64)
#define FC_LISTS (FC_NW * 16)     // key lists per query: (wave, lane column)
#define FC_RPW (FC_QB / FC_NW)    // queries each wave selects for

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

// Pack centroids into bf16 hi/lo chunks in the order the MFMA lanes read
// them, so each (tile, half, slice) is one contiguous 1 KB load: chunk
// Cb[(((tile * 2 + h) * DT + t) * 4 + g) * 16 + c % 16], tile = c / 16, holds
// the eight dimensions 32 t + 8 g .. + 7 of centroid c (h = 0: hi, 1: lo),
// zero beyond d and for the padding centroids L .. Lp - 1 (Lp = L rounded up
// to an even number of rounds of FC_NW tiles, so tile loads need no bounds).
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

// L padded to an even number of rounds of FC_NW tiles (every wave has the
// same tiles, in pairs)
static int fc_padded_lists(int L) { return (L + 2 * FC_LISTS - 1) / (2 * FC_LISTS) * (2 * FC_LISTS); }

size_t coarse_bf16_pack_chunks(int L, int d) { return (size_t)fc_padded_lists(L) * ((d + 31) / 32) * 8; }

void launch_coarse_bf16_pack(const float* C, int L, int d, uint4* Cb, hipStream_t s) {
    const int DT = (d + 31) / 32, Lp = fc_padded_lists(L);
    const size_t n = (size_t)Lp * DT * 4;
    if (n == 0) return;
    hipLaunchKernelGGL(coarse_bf16_pack_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, C,
                       L, Lp, d, DT, Cb);
}

// Keys per list and candidates per query: a list holds 1/128 of the
// centroids, so J of them cover the Pe nearest unless more than J of those
// (and of the lists within the error margin) share one list: rare at these J
// (about 1e-4 of queries at Pe = 32, J = 6).  Up to 320 candidates above 32
// probes (a few hundred exactly tied lists still take the candidate path).
__host__ __device__ constexpr int fc_cap(int J) { return J <= 6 ? 128 : 320; }

// Dynamic LDS of the fused kernel: the query tile [FC_QB][fc_tile_stride(d)]
// floats (kept for the exact rescoring); one region used first for the list
// maxima [FC_QB][FC_LISTS] and the MFMA operands, then for the candidate
// lists [FC_QB][CAP] and their keys [FC_QB][CAP] (later the lists to rescore
// and their scores); then ten [FC_QB] arrays of per-query values.
__host__ __device__ inline int fc_tile_stride(int d) { return (d & ~3) + 4; }  // 16-byte rows
__host__ __device__ inline size_t fc_tile_bytes(int d) { return (size_t)FC_QB * fc_tile_stride(d) * 4; }
__host__ __device__ inline size_t fc_work_bytes(int J, int DT) {
    // the maxima and, until the pass, the MFMA operands [FC_QBW][DT][2][64] after them
    const size_t mx = (size_t)FC_QB * FC_LISTS * 4 + (size_t)FC_QBW * DT * 2 * 64 * 16;
    const size_t cand = 2 * (size_t)FC_QB * fc_cap(J) * 4;
    return mx > cand ? mx : cand;
}
__host__ __device__ inline size_t fc_lds_bytes(int d, int J, int DT) {
    return fc_tile_bytes(d) + fc_work_bytes(J, DT) + 10 * FC_QB * 4;
}

// One pass of bf16x3 products over every centroid.  Wave h takes the
// 16-centroid tiles h, h + FC_NW, ... (nt of them; Cb is padded to whole rounds
// of FC_NW tiles, so no load needs a bound) and, for its i-th tile, hands
// acc[b] = Q_b . C_tile^T (16 x 16, query block b) to epi(acc, i).  The B
// operands come straight from L2: each (tile, half, 32-dimension slice) is
// 1 KB, one 16-byte chunk per lane, and slice t of the next tile is loaded as
// soon as the current tile's products with slice t are issued (with DB,
// slice t of the tile after next, into a second register set).
template <int DT>
__device__ __forceinline__ __amdgpu_buffer_rsrc_t fc_rsrc(const uint4* Cb, int nt) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<uint4*>(Cb), (short)0, nt * FC_NW * 2 * DT * 1024,
                                             0x00020000);
}

// slice T of tile TILE into register set S
#define FC_LOAD(S, TILE, T)                                                                              \
    bh[S][T] = __builtin_amdgcn_raw_buffer_load_b128(rsrc, lofs, (uint32_t)((((TILE) * 2 + 0) * DT + (T)) * 1024), 0); \
    bl[S][T] = __builtin_amdgcn_raw_buffer_load_b128(rsrc, lofs, (uint32_t)((((TILE) * 2 + 1) * DT + (T)) * 1024), 0);

// The loads of the wave's first tiles (two register sets with DB: tiles 0
// and 1; else tile 0), issued before fc_pass so they travel while the
// workgroup prepares its queries.
template <int DT, bool DB>
__device__ __forceinline__ void fc_prefetch(const uint4* __restrict__ Cb, int nt, int h, u32x4 (&bh)[DB ? 2 : 1][DT],
                                            u32x4 (&bl)[DB ? 2 : 1][DT]) {
    const __amdgpu_buffer_rsrc_t rsrc = fc_rsrc<DT>(Cb, nt);
    const uint32_t lofs = (uint32_t)(threadIdx.x & 63) * 16u;
#pragma unroll
    for (int t = 0; t < DT; t++) { FC_LOAD(0, h, t) }
    if (DB) {
#pragma unroll
        for (int t = 0; t < DT; t++) { FC_LOAD(DB ? 1 : 0, FC_NW * (nt > 1 ? 1 : 0) + h, t) }
    }
}

template <int DT, bool DB, typename Epi>
__device__ __forceinline__ void fc_pass(const uint4* __restrict__ Cb, int nt, int h, u32x4 (&bh)[DB ? 2 : 1][DT],
                                        u32x4 (&bl)[DB ? 2 : 1][DT], const u32x4 (&ah)[FC_QBW][DT],
                                        const u32x4 (&al)[FC_QBW][DT], Epi epi) {
    const __amdgpu_buffer_rsrc_t rsrc = fc_rsrc<DT>(Cb, nt);
    const uint32_t lofs = (uint32_t)(threadIdx.x & 63) * 16u;
    // two register sets (DB): tile i + 2 loads into the set tile i used;
    // else one, and tile i + 1 loads into it
    constexpr int NS = DB ? 2 : 1, AHEAD = DB ? 2 : 1;
    // tile i from set S; set S then loads tile i + AHEAD (the last ones
    // reload themselves: in bounds, never used)
#define FC_TILE(S, I, M)                                                                                 \
    {                                                                                                    \
        const int i_ = (I);                                                                              \
        const int nxt = FC_NW * (i_ + AHEAD < nt ? i_ + AHEAD : i_) + h;                                 \
        floatx4 acc[FC_QBW];                                                                             \
        _Pragma("unroll") for (int b = 0; b < FC_QBW; b++) acc[b] = floatx4{0.f, 0.f, 0.f, 0.f};         \
        _Pragma("unroll") for (int t = 0; t < DT; t++) {                                                 \
            const bf16x8 b_h = __builtin_bit_cast(bf16x8, bh[S][t]);                                     \
            const bf16x8 b_l = __builtin_bit_cast(bf16x8, bl[S][t]);                                     \
            _Pragma("unroll") for (int b = 0; b < FC_QBW; b++)                                           \
                acc[b] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, ah[b][t]), b_l, acc[b], 0, 0, 0); \
            _Pragma("unroll") for (int b = 0; b < FC_QBW; b++)                                           \
                acc[b] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, al[b][t]), b_h, acc[b], 0, 0, 0); \
            _Pragma("unroll") for (int b = 0; b < FC_QBW; b++)                                           \
                acc[b] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, ah[b][t]), b_h, acc[b], 0, 0, 0); \
            FC_LOAD(S, nxt, t)                                                                           \
        }                                                                                                \
        epi(acc, i_, M);                                                                                 \
    }
    // only the last round may reach past L (M: the epilogue masks)
    if (DB) {  // nt is even
        for (int i = 0; i + 2 < nt; i += 2) {
            FC_TILE(0, i, false)
            FC_TILE(NS - 1, i + 1, false)
        }
        FC_TILE(0, nt - 2, true)
        FC_TILE(NS - 1, nt - 1, true)
    } else {
        for (int i = 0; i + 1 < nt; i++) FC_TILE(0, i, false)
        FC_TILE(0, nt - 1, true)
    }
#undef FC_TILE
}
#undef FC_LOAD

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

// Inclusive prefix sum over the 16 lanes of each DPP row (row_shr 1, 2, 4, 8;
// lanes shifted in from outside the row add 0).
__device__ __forceinline__ uint32_t prefix16(uint32_t x) {
    x += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, 0x111, 0xF, 0xF, false);
    x += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, 0x112, 0xF, 0xF, false);
    x += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, 0x114, 0xF, 0xF, false);
    x += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, 0x118, 0xF, 0xF, false);
    return x;
}

// Element pos (wave-uniform) of a wave-held array, element e * 64 + lane in v[e].
template <int E>
__device__ __forceinline__ float wave_at(const float (&v)[E], int pos) {
    float x = v[0];
#pragma unroll
    for (int e = 1; e < E; e++) x = (pos >> 6) == e ? v[e] : x;
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), pos & 63));
}

// Classification of one query's n <= 64 E candidates (lists ids[t], keys
// keys[t]), one wave.  Keys are sorted descending with the slot t in their
// low SB bits (so each is truncated by under 2^SB ulps, ulp <= `ulp`); score
// s = 3 - key is then within m = mar + 2^SB ulp of the reference score
// 1 - dot, so with m2 = 2 m a candidate is surely among the Pe smallest when s + m2 is below
// the score at position Pe (the n - Pe candidates from there on all trail it
// for sure), and surely not when s - m2 is above the score at position Pe - 1.
// The sure members are the first `in` positions and are written to pr at
// their position (nearest first); the `un` uncertain ones follow them and are
// copied to unc in that order.  `ordered`: every candidate is uncertain.
// Reads all keys before it writes unc, which may overlay them.
template <int E>
__device__ __forceinline__ void fc_classify_sorted(const uint32_t (&sk)[E], const uint32_t* ids, uint32_t* unc,
                                                   uint32_t* pr, uint32_t n, int Pe, float mar, float ulp,
                                                   int ordered, uint32_t& in, uint32_t& un) {
    const int lane = threadIdx.x & 63;
    constexpr int SB = E == 1 ? 6 : E == 2 ? 7 : E == 4 ? 8 : 9;
    constexpr uint32_t SM = (1u << SB) - 1u;
    const float m2 = 2.0f * (mar + (float)(1u << SB) * ulp);
    float cs[E];
#pragma unroll
    for (int e = 0; e < E; e++) cs[e] = 3.0f - fkey_to_float(~(sk[e] | SM));
    float lo_m = 3.0e38f, hi_m = 3.0e38f;  // every candidate a sure member (n <= Pe)
    if (ordered) {
        lo_m = -3.0e38f;  // none sure either way
    } else if (n > (uint32_t)Pe) {
        lo_m = wave_at<E>(cs, Pe) - m2;
        hi_m = wave_at<E>(cs, Pe - 1) + m2;
    }
    in = 0;
    un = 0;
    uint32_t cls[E];  // 1 sure member, 2 to rescore, 0 out
#pragma unroll
    for (int e = 0; e < E; e++) {
        const uint32_t t = e * 64 + lane;
        cls[e] = t >= n ? 0u : lo_m > cs[e] ? 1u : hi_m < cs[e] ? 0u : 2u;
        in += (uint32_t)__popcll(__ballot(cls[e] == 1u));
        un += (uint32_t)__popcll(__ballot(cls[e] == 2u));
    }
#pragma unroll
    for (int e = 0; e < E; e++) {
        const uint32_t t = e * 64 + lane;
        if (cls[e] == 1u) pr[t] = ids[sk[e] & SM];
        if (cls[e] == 2u) unc[t - in] = ids[sk[e] & SM];
    }
}

template <int E>
__device__ __forceinline__ void fc_classify(const uint32_t* ids, const float* keys, uint32_t* unc, uint32_t* pr,
                                            uint32_t n, int Pe, float mar, float ulp, int ordered, uint32_t& in,
                                            uint32_t& un) {
    const int lane = threadIdx.x & 63;
    constexpr int SB = E == 1 ? 6 : E == 2 ? 7 : E == 4 ? 8 : 9;
    constexpr uint32_t SM = (1u << SB) - 1u;
    uint32_t sk[E];
#pragma unroll
    for (int e = 0; e < E; e++) {
        const uint32_t t = e * 64 + lane;
        sk[e] = t < n ? (~fkey(keys[t]) & ~SM) | t : ~0u;
    }
    wave_sort_u32<E>(sk);
    fc_classify_sorted<E>(sk, ids, unc, pr, n, Pe, mar, ulp, ordered, in, un);
}

// One sequential dot (src/simd.rs:88-91 order) with the whole centroid row
// (d <= 32 DT floats) loaded before the sum starts; q in LDS.  Rows 16-byte
// aligned when d % 4 == 0 (else one float at a time).
template <int DT>
__device__ __forceinline__ float fc_seq_dot(const float* q, const float* __restrict__ cr, int d) {
    float out = 0.0f;
    if (d & 3) {
        for (int j = 0; j < d; j++) out = __fadd_rn(out, __fmul_rn(q[j], cr[j]));
        return out;
    }
    float4 v[8 * DT];
#pragma unroll
    for (int i = 0; i < 8 * DT; i++)
        v[i] = 4 * i < d ? reinterpret_cast<const float4*>(cr)[i] : make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
    for (int i = 0; i < 8 * DT; i++) {
        // past d: 0 * 0 adds nothing
        const float4 a = 4 * i < d ? reinterpret_cast<const float4*>(q)[i] : make_float4(0.f, 0.f, 0.f, 0.f);
        out = __fadd_rn(out, __fmul_rn(a.x, v[i].x));
        out = __fadd_rn(out, __fmul_rn(a.y, v[i].y));
        out = __fadd_rn(out, __fmul_rn(a.z, v[i].z));
        out = __fadd_rn(out, __fmul_rn(a.w, v[i].w));
    }
    return out;
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
    const float* __restrict__ Q, int nq, int d, const uint4* __restrict__ Cb, int L, int nt, float cmax,
    int Pe, int P, int IB, int normalize, int ordered, float* __restrict__ qn_out, float* __restrict__ qnorm_out,
    const float* __restrict__ C, uint32_t* __restrict__ probe, uint32_t* __restrict__ flag_list,
    uint32_t* __restrict__ flag_count, uint32_t* __restrict__ qbad, unsigned int* __restrict__ nbad) {
    extern __shared__ __align__(16) char smem[];
    constexpr int CAP = fc_cap(J);
    const int tid = threadIdx.x, lane = tid & 63, g = lane >> 4, c = lane & 15;
    const int h = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int q0 = blockIdx.x * FC_QB;
    const int rows = min(FC_QB, nq - q0);
    const int st = fc_tile_stride(d);
    float* tile = reinterpret_cast<float*>(smem);
    char* work = smem + fc_tile_bytes(d);
    float* mx = reinterpret_cast<float*>(work);                   // [FC_QB][FC_LISTS] list maxima
    uint32_t* cid = reinterpret_cast<uint32_t*>(work);           // [FC_QB][CAP] candidate lists
    float* ckey = reinterpret_cast<float*>(work) + FC_QB * CAP;  // [FC_QB][CAP] their keys
    float* rv = reinterpret_cast<float*>(work + fc_work_bytes(J, DT));
    float* snorm = rv;               // the norm divided by (0: rows used as given)
    float* sbnd = rv + FC_QB;        // bound on ||q||
    float* skthr = rv + 2 * FC_QB;   // candidate threshold on the keys
    float* smar = rv + 3 * FC_QB;    // margin of the candidates' scores
    float* sulp = rv + 7 * FC_QB;    // bound on the ulp of the keys
    uint32_t* sin = reinterpret_cast<uint32_t*>(rv + 8 * FC_QB);  // probes written: the sure members
    uint32_t* sun = reinterpret_cast<uint32_t*>(rv + 9 * FC_QB);  // lists left to rescore
    uint32_t* scnt = reinterpret_cast<uint32_t*>(rv + 4 * FC_QB);   // candidates
    uint32_t* sbad = reinterpret_cast<uint32_t*>(rv + 5 * FC_QB);   // holds a NaN or an infinity
    uint32_t* sover = reinterpret_cast<uint32_t*>(rv + 6 * FC_QB);  // candidate set may be incomplete

    constexpr bool DB = !(DT == 4 && J == 8);  // a second register set fits
    u32x4 bh[DB ? 2 : 1][DT], bl[DB ? 2 : 1][DT];
    fc_prefetch<DT, DB>(Cb, nt, h, bh, bl);

    // ---- normalise (search.rs:55-62): sequential sum of squares per row.  A
    // row holding a NaN or an infinity is searched as the zero vector, marked
    // in qbad and counted in *nbad (its result row becomes padding).
    if (tid < FC_QB) {
        scnt[tid] = 0u;
        sbad[tid] = 0u;
        sover[tid] = 0u;
    }
    __syncthreads();
    const float* src = Q + (size_t)q0 * d;
    // thread -> (rows r0, r0 + rstep, ..., one column): one division per thread
    const bool vec = (d & 3) == 0 && (reinterpret_cast<uintptr_t>(src) & 15) == 0 &&
                     (!normalize || (reinterpret_cast<uintptr_t>(qn_out) & 15) == 0);
    const int wrow = vec ? d >> 2 : d;  // items per row
    const int rstep = FC_THREADS / wrow;
    const int r0 = tid / wrow, jc = tid - r0 * wrow;
    const uint32_t ex = 0x7f800000u;
    if (r0 < rstep) {
        if (vec && rstep * 3 >= FC_QB) {  // d > 64: every load in flight at once
            float4 v[3];
#pragma unroll
            for (int k = 0; k < 3; k++) {
                const int r = r0 + k * rstep;
                v[k] = r < rows ? reinterpret_cast<const float4*>(src + (size_t)r * d)[jc]
                                : make_float4(0.f, 0.f, 0.f, 0.f);
            }
#pragma unroll
            for (int k = 0; k < 3; k++) {
                const int r = r0 + k * rstep;
                if (r < FC_QB) {
                    if ((__float_as_uint(v[k].x) & ex) == ex || (__float_as_uint(v[k].y) & ex) == ex ||
                        (__float_as_uint(v[k].z) & ex) == ex || (__float_as_uint(v[k].w) & ex) == ex)
                        sbad[r] = 1u;
                    *reinterpret_cast<float4*>(tile + r * st + 4 * jc) = v[k];
                }
            }
        } else if (vec) {
            for (int r = r0; r < FC_QB; r += rstep) {
                const float4 v = r < rows ? reinterpret_cast<const float4*>(src + (size_t)r * d)[jc]
                                          : make_float4(0.f, 0.f, 0.f, 0.f);
                if ((__float_as_uint(v.x) & ex) == ex || (__float_as_uint(v.y) & ex) == ex ||
                    (__float_as_uint(v.z) & ex) == ex || (__float_as_uint(v.w) & ex) == ex)
                    sbad[r] = 1u;
                *reinterpret_cast<float4*>(tile + r * st + 4 * jc) = v;
            }
        } else {
            for (int r = r0; r < FC_QB; r += rstep) {
                const float v = r < rows ? src[(size_t)r * d + jc] : 0.0f;
                if ((__float_as_uint(v) & ex) == ex) sbad[r] = 1u;
                tile[r * st + jc] = v;
            }
        }
    }
    __syncthreads();
    if (tid < FC_QB) {
        const float* xr = tile + tid * st;
        const bool bad = sbad[tid] != 0u;
        float s = 0.0f;
        if (!bad) {
            if ((d & 3) == 0) {
                // all of the row's loads first, then the sequential sum
                // (the zeros past d add nothing)
#pragma unroll
                for (int t = 0; t < DT; t++) {
                    float4 v[8];
#pragma unroll
                    for (int i = 0; i < 8; i++)
                        v[i] = 32 * t + 4 * i < d ? *reinterpret_cast<const float4*>(xr + 32 * t + 4 * i)
                                                  : make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
                    for (int i = 0; i < 8; i++) {
                        s = __fadd_rn(s, __fmul_rn(v[i].x, v[i].x));
                        s = __fadd_rn(s, __fmul_rn(v[i].y, v[i].y));
                        s = __fadd_rn(s, __fmul_rn(v[i].z, v[i].z));
                        s = __fadd_rn(s, __fmul_rn(v[i].w, v[i].w));
                    }
                }
            } else {
                for (int j = 0; j < d; j++) s = __fadd_rn(s, __fmul_rn(xr[j], xr[j]));
            }
        }
        if (bad && nbad) atomicAdd(nbad, 1u);
        if (qbad && tid < rows) qbad[q0 + tid] = bad ? 1u : 0u;
        const float nrm = sqrtf(s);
        // without normalisation the rows are used as given; the bound is ||x||
        snorm[tid] = normalize ? nrm : 0.0f;
        sbnd[tid] = normalize && nrm > 1e-10f ? 1.0001f : nrm * 1.0001f + 1e-30f;
        if (tid < rows && qnorm_out) qnorm_out[q0 + tid] = sbnd[tid];
    }
    __syncthreads();
    // divide by the norm (zeroing the marked rows), write qn, and split each
    // 8-dimension group into its bf16 hi/lo MFMA operands, kept in LDS past
    // the maxima: As[((b * DT + t) * 2 + half) * 64 + 16 g + c] holds
    // dimensions 32 t + 8 g .. + 7 of query 16 b + c
    u32x4* As = reinterpret_cast<u32x4*>(work + (size_t)FC_QB * FC_LISTS * 4);
    {
        constexpr int G8 = 4 * DT;  // 8-dimension groups per row
        const bool v8 = (d & 7) == 0 && (!normalize || (reinterpret_cast<uintptr_t>(qn_out) & 15) == 0);
        for (int k = tid; k < FC_QB * G8; k += FC_THREADS) {
            const int r = k / G8, g8 = k - r * G8, j0 = 8 * g8;
            const float nrm = snorm[r];
            const bool zero = sbad[r] != 0u, div = nrm > 1e-10f;
            float* tr = tile + r * st + j0;
            float x[8];
            if (v8) {
                const float4 lo = j0 < d ? reinterpret_cast<const float4*>(tr)[0] : make_float4(0.f, 0.f, 0.f, 0.f);
                const float4 hi = j0 < d ? reinterpret_cast<const float4*>(tr)[1] : make_float4(0.f, 0.f, 0.f, 0.f);
                x[0] = lo.x; x[1] = lo.y; x[2] = lo.z; x[3] = lo.w;
                x[4] = hi.x; x[5] = hi.y; x[6] = hi.z; x[7] = hi.w;
            } else {
#pragma unroll
                for (int i = 0; i < 8; i++) x[i] = j0 + i < d ? tr[i] : 0.0f;
            }
#pragma unroll
            for (int i = 0; i < 8; i++) x[i] = zero ? 0.0f : div ? x[i] / nrm : x[i];
            if (v8) {
                if (j0 < d) {
                    const float4 lo = make_float4(x[0], x[1], x[2], x[3]), hi = make_float4(x[4], x[5], x[6], x[7]);
                    reinterpret_cast<float4*>(tr)[0] = lo;
                    reinterpret_cast<float4*>(tr)[1] = hi;
                    if (normalize && r < rows) {
                        float4* qo = reinterpret_cast<float4*>(qn_out + (size_t)(q0 + r) * d + j0);
                        qo[0] = lo;
                        qo[1] = hi;
                    }
                }
            } else {
#pragma unroll
                for (int i = 0; i < 8; i++)
                    if (j0 + i < d) {
                        tr[i] = x[i];
                        if (normalize && r < rows) qn_out[(size_t)(q0 + r) * d + j0 + i] = x[i];
                    }
            }
            uint32_t hb[8], lb[8];
#pragma unroll
            for (int i = 0; i < 8; i++) bf16_split(x[i], hb[i], lb[i]);
            const int slot = ((r >> 4) * DT + (g8 >> 2)) * 2 * 64 + 16 * (g8 & 3) + (r & 15);
            As[slot] = u32x4{hb[0] | hb[1] << 16, hb[2] | hb[3] << 16, hb[4] | hb[5] << 16, hb[6] | hb[7] << 16};
            As[slot + 64] = u32x4{lb[0] | lb[1] << 16, lb[2] | lb[3] << 16, lb[4] | lb[5] << 16, lb[6] | lb[7] << 16};
        }
    }
    __syncthreads();
    u32x4 ah[FC_QBW][DT], al[FC_QBW][DT];
#pragma unroll
    for (int b = 0; b < FC_QBW; b++)
#pragma unroll
        for (int t = 0; t < DT; t++) {
            ah[b][t] = As[(b * DT + t) * 2 * 64 + lane];
            al[b][t] = As[(b * DT + t) * 2 * 64 + 64 + lane];
        }

    // ---- the pass: every (lane, query 16 b + 4 g + r) keeps the J largest
    // keys k = (a + 2) with the low IB mantissa bits replaced by the wave's
    // tile number i (a = approximate q.c; list = 16 (FC_NW i + h) + c).
    const uint32_t kmask = ~((1u << IB) - 1u);
    float top[FC_QBW][4][J];
#pragma unroll
    for (int b = 0; b < FC_QBW; b++)
#pragma unroll
        for (int r = 0; r < 4; r++)
#pragma unroll
            for (int j = 0; j < J; j++) top[b][r][j] = -3.0e38f;  // below every key
    fc_pass<DT, DB>(Cb, nt, h, bh, bl, ah, al, [&](const floatx4 (&acc)[FC_QBW], int i, bool masked) {
        const bool valid = !masked || (FC_NW * i + h) * 16 + c < L;
        // the tile number in a vector register, so mask and insert are one
        // v_and_or_b32 (a single scalar operand per instruction)
        const uint32_t ti = (uint32_t)__builtin_amdgcn_update_dpp(0, i, 0xE4, 0xF, 0xF, false);
#pragma unroll
        for (int b = 0; b < FC_QBW; b++)
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const float k = __uint_as_float((__float_as_uint(acc[b][r] + 2.0f) & kmask) | ti);
                top_insert<J>(top[b][r], valid ? k : -3.0e38f);
            }
    });

    // ---- threshold: the Pe-th largest of a query's 128 list maxima, T,
    // bounds its Pe-th largest key from below.  Keys are within E of a + 2 and
    // a within eps of the reference's dot, so every list among the Pe exact
    // nearest has a key >= T - 2E - 2 eps (taken with a factor 1.25 and a few
    // ulps to spare); in each list those keys are a prefix.
#pragma unroll
    for (int b = 0; b < FC_QBW; b++)
#pragma unroll
        for (int r = 0; r < 4; r++) mx[(b * 16 + 4 * g + r) * FC_LISTS + h * 16 + c] = top[b][r][0];
    __syncthreads();
    const float u = 5.9604645e-08f;
    {
        // radix selection, all of the wave's queries at once: the largest t
        // with at least Pe maxima >= t is the Pe-th largest; stopped at bit
        // 8, t is below it by under 256 units of the key order (ulps), still
        // a bound with Pe maxima at or above it
        uint32_t v0[FC_RPW], v1[FC_RPW], res[FC_RPW];
#pragma unroll
        for (int i = 0; i < FC_RPW; i++) {
            const int row = h + FC_NW * i;
            const bool act = row < rows;
            v0[i] = act ? fkey(mx[row * FC_LISTS + lane]) : 0u;
            v1[i] = act ? fkey(mx[row * FC_LISTS + 64 + lane]) : 0u;
            res[i] = 0u;
        }
        if (Pe <= 32) {
            // the maxima of list pairs (l, l + 64): still Pe distinct lists
            // at or above t, one comparison per bit
#pragma unroll
            for (int i = 0; i < FC_RPW; i++) v0[i] = max(v0[i], v1[i]);
            for (int bit = 31; bit >= 8; bit--) {
#pragma unroll
                for (int i = 0; i < FC_RPW; i++) {
                    const uint32_t cand = res[i] | (1u << bit);
                    res[i] = (uint32_t)__popcll(__ballot(v0[i] >= cand)) >= (uint32_t)Pe ? cand : res[i];
                }
            }
        } else {
            for (int bit = 31; bit >= 8; bit--) {
#pragma unroll
                for (int i = 0; i < FC_RPW; i++) {
                    const uint32_t cand = res[i] | (1u << bit);
                    const uint32_t cnt =
                        (uint32_t)__popcll(__ballot(v0[i] >= cand)) + (uint32_t)__popcll(__ballot(v1[i] >= cand));
                    res[i] = cnt >= (uint32_t)Pe ? cand : res[i];
                }
            }
        }
        if (lane < FC_RPW) {
            uint32_t tk = res[0];
#pragma unroll
            for (int i = 1; i < FC_RPW; i++) tk = lane == i ? res[i] : tk;
            const int row = h + FC_NW * lane;
            if (row < rows) {
                const float T = fkey_to_float(tk);
                const float qb_norm = sbnd[row];
                const float qc = qb_norm * cmax;
                // packing: < 2^IB ulps of a + 2 plus half an ulp of its
                // rounding; every |a + 2| <= qc + 2 < ub (a power of two) has
                // ulp <= ub u
                const float ub = __uint_as_float((__float_as_uint(qc + 2.0f) & 0x7f800000u) + 0x00800000u);
                const float E = ((float)(1u << IB) + 0.5f) * ub * u;
                const float eps = coarse_eps_bf16(d, qb_norm, cmax);
                skthr[row] = T - (2.0f * E + 2.5f * eps + 8.0f * ub * u);
                // the reference score 1 - dot is within this of 3 - key
                smar[row] = E + 1.25f * eps + 4.0f * ub * u;
                sulp[row] = ub * u;
            }
        }
    }
    __syncthreads();

    // ---- candidates: the keys >= the threshold, to LDS [row][CAP].  A list
    // whose J-th key passes may have dropped one, and a query holds at most
    // CAP: the query is then marked.
    {
        uint32_t nn[FC_QBW * 4], base[FC_QBW * 4];
#pragma unroll
        for (int b = 0; b < FC_QBW; b++)
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const int row = b * 16 + 4 * g + r;
                const bool act = row < rows;
                const float kthr = act ? skthr[row] : 3.0e38f;
                uint32_t n = 0;
#pragma unroll
                for (int j = 0; j < J; j++) n += top[b][r][j] >= kthr ? 1u : 0u;
                nn[b * 4 + r] = n;
                base[b * 4 + r] = prefix16(n);
                if (act && top[b][r][J - 1] >= kthr) sover[row] = 1u;
            }
        // the last lane of each group reserves the group's slots: every
        // reservation issued before the first result is read
        uint32_t o[FC_QBW * 4];
#pragma unroll
        for (int k = 0; k < FC_QBW * 4; k++) {
            const int row = (k >> 2) * 16 + 4 * g + (k & 3);
            o[k] = 0;
            if (row < rows && c == 15 && base[k] > 0) o[k] = atomicAdd(&scnt[row], base[k]);
        }
#pragma unroll
        for (int k = 0; k < FC_QBW * 4; k++)
            base[k] = (uint32_t)__shfl((int)o[k], (lane & 48) | 15, 64) + base[k] - nn[k];
#pragma unroll
        for (int b = 0; b < FC_QBW; b++)
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const int row = b * 16 + 4 * g + r;
                const uint32_t n = nn[b * 4 + r], o = base[b * 4 + r];
#pragma unroll
                for (int j = 0; j < J; j++) {
                    if (__ballot((uint32_t)j < n) == 0) break;  // no lane has a j-th candidate
                    if ((uint32_t)j < n && o + j < (uint32_t)CAP) {
                        const uint32_t ti = __float_as_uint(top[b][r][j]) & ~kmask;
                        cid[row * CAP + o + j] = 16u * (FC_NW * ti + (uint32_t)h) + (uint32_t)c;
                        ckey[row * CAP + o + j] = top[b][r][j];
                    }
                }
            }
    }
    __syncthreads();

    // ---- the selection, wave h for queries h, h + FC_NW, ...: the sure
    // members go out at once, the uncertain ones are rescored with the
    // reference's sequential dot against the query as searched
    // (distance.rs:104-109) and ranked by (score, list) for the places left.
    uint32_t* uid = reinterpret_cast<uint32_t*>(ckey);  // lists to rescore, over the keys
    {
        uint32_t nr[FC_RPW];  // candidates of each query (0: nothing to select)
        uint32_t sk[FC_RPW];  // keys of the queries with at most 64, sorted together
        uint32_t big = 0;     // queries with more than 64
#pragma unroll
        for (int i = 0; i < FC_RPW; i++) {
            const int row = h + FC_NW * i;
            uint32_t n = 0;
            if (row < rows) {
                n = scnt[row];
                if (sover[row] || n > (uint32_t)CAP) {  // may be incomplete: the exact fallback
                    if (lane == 0) flag_list[atomicAdd(flag_count, 1u)] = (uint32_t)(q0 + row);
                    n = 0;
                }
                if (lane == 0) {
                    sin[row] = (uint32_t)Pe;
                    sun[row] = 0u;
                }
            }
            nr[i] = n;
            big |= n > 64u ? 1u << i : 0u;
            sk[i] = (uint32_t)lane < n && n <= 64u ? (~fkey(ckey[row * CAP + lane]) & ~63u) | (uint32_t)lane : ~0u;
        }
        wave_sort_u32_sep<FC_RPW>(sk);
#pragma unroll
        for (int i = 0; i < FC_RPW; i++) {
            const int row = h + FC_NW * i;
            const uint32_t n = nr[i];
            if (n > 0 && n <= 64) {
                uint32_t in, un;
                const uint32_t s1[1] = {sk[i]};
                fc_classify_sorted<1>(s1, cid + row * CAP, uid + row * CAP, probe + (size_t)(q0 + row) * P, n,
                                      Pe, smar[row], sulp[row], ordered, in, un);
                if (lane == 0) {
                    sin[row] = in;
                    sun[row] = in < (uint32_t)Pe ? un : 0u;
                }
            }
        }
#pragma unroll 1
        for (int i = 0; i < FC_RPW; i++) {
            if (!(big >> i & 1u)) continue;
            const int row = h + FC_NW * i;
            const uint32_t n = scnt[row];
            uint32_t* pr = probe + (size_t)(q0 + row) * P;
            const uint32_t* ids = cid + row * CAP;
            const float* keys = ckey + row * CAP;
            uint32_t* unc = uid + row * CAP;
            const float mar = smar[row], ulp = sulp[row];
            uint32_t in, un;
            if (CAP <= 128 || n <= 128) fc_classify<2>(ids, keys, unc, pr, n, Pe, mar, ulp, ordered, in, un);
            else if (n <= 256) fc_classify<4>(ids, keys, unc, pr, n, Pe, mar, ulp, ordered, in, un);
            else fc_classify<8>(ids, keys, unc, pr, n, Pe, mar, ulp, ordered, in, un);
            if (lane == 0) {
                sin[row] = in;
                sun[row] = in < (uint32_t)Pe ? un : 0u;
            }
        }
    }
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
    __builtin_amdgcn_wave_barrier();
    // the lists to rescore, numbered in query order, one per lane; the
    // scores go over the candidate lists
    uint32_t rbeg[FC_RPW + 1];
    rbeg[0] = 0;
#pragma unroll
    for (int i = 0; i < FC_RPW; i++) {
        const int row = h + FC_NW * i;
        rbeg[i + 1] = rbeg[i] + (row < rows ? sun[row] : 0u);
    }
    const uint32_t tot = rbeg[FC_RPW];
    for (uint32_t b0 = 0; b0 < tot; b0 += 64) {
        const uint32_t x = b0 + lane;
        int row = h;
        uint32_t beg = 0;
#pragma unroll
        for (int i = 1; i < FC_RPW; i++)
            if (x >= rbeg[i]) {
                row = h + FC_NW * i;
                beg = rbeg[i];
            }
        if (x < tot) {
            const uint32_t at = (uint32_t)row * CAP + (x - beg);
            const float dot = fc_seq_dot<DT>(tile + row * st, C + (size_t)uid[at] * d, d);
            cid[at] = fkey(1.0f - dot);
        }
    }
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
    __builtin_amdgcn_wave_barrier();
#pragma unroll 1
    for (int i = 0; i < FC_RPW; i++) {
        const int row = h + FC_NW * i;
        if (row >= rows) break;
        const uint32_t n = sun[row];
        if (n == 0) continue;  // nothing left to rank or marked
        const uint32_t* cr = uid + row * CAP;
        const uint32_t* sr = cid + row * CAP;
        const uint32_t rin = sin[row];
        uint32_t* pr = probe + (size_t)(q0 + row) * P + rin;
        const int need = Pe - (int)rin;
        if (n <= 16) {
            // a few: each one's rank by counting
            const bool mine = (uint32_t)lane < n;
            const uint64_t kv = mine ? ((uint64_t)sr[lane] << 32) | cr[lane] : ~0ull;
            uint32_t rank = 0;
            for (uint32_t j = 0; j < n; j++) {
                const uint64_t o = ((uint64_t)(uint32_t)__builtin_amdgcn_readlane((int)(kv >> 32), (int)j) << 32) |
                                   (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)kv, (int)j);
                rank += o < kv ? 1u : 0u;
            }
            if (mine && rank < (uint32_t)need) pr[rank] = (uint32_t)kv;
        } else if (n <= 64) {
            fc_select_row<1>(cr, sr, n, need, pr);
        } else if (CAP <= 128 || n <= 128) {
            fc_select_row<2>(cr, sr, n, need, pr);
        } else if (n <= 256) {
            fc_select_row<4>(cr, sr, n, need, pr);
        } else {
            fc_select_row<8>(cr, sr, n, need, pr);
        }
    }
}

// Keys per list: 4 up to 8 probes, 6 up to 32, 8 above.
static int fc_keys(int Pe) { return Pe <= 8 ? 4 : Pe <= 32 ? 6 : 8; }

bool coarse_fused_supported(int d, int P) { return d >= 1 && d <= 128 && P >= 1 && P <= 64; }

static int fc_tiles_per_wave(int L) { return fc_padded_lists(L) / FC_LISTS; }

template <int DT, int J>
static void launch_fused(const float* Q, int nq, int d, const uint4* Cb, int L, float cmax, int Pe, int P,
                         int normalize, int ordered, float* qn, float* qnorm, const float* C, uint32_t* probe,
                         uint32_t* flag_list, uint32_t* flag_count, hipStream_t s, uint32_t* qbad,
                         unsigned int* nbad) {
    const size_t lds = fc_lds_bytes(d, J, DT);
    const int nt = fc_tiles_per_wave(L);
    // index bits: a wave's tile numbers 0 .. nt - 1 < 2^IB
    int IB = 0;
    while ((1 << IB) < nt) IB++;
    auto k = coarse_fused_kernel<DT, J>;
    ensure_dyn_lds((const void*)k, lds);
    hipLaunchKernelGGL(k, dim3((nq + FC_QB - 1) / FC_QB), dim3(FC_THREADS), lds, s, Q, nq, d, Cb, L, nt, cmax,
                       Pe, P, IB, normalize, ordered, qn, qnorm, C, probe, flag_list, flag_count, qbad, nbad);
}

template <int DT>
static void launch_fused_j(const float* Q, int nq, int d, const uint4* Cb, int L, float cmax, int Pe, int P,
                           int normalize, int ordered, float* qn, float* qnorm, const float* C, uint32_t* probe,
                           uint32_t* flag_list, uint32_t* flag_count, hipStream_t s, uint32_t* qbad,
                           unsigned int* nbad) {
#define FC_J(JV) launch_fused<DT, JV>(Q, nq, d, Cb, L, cmax, Pe, P, normalize, ordered, qn, qnorm, C, probe, \
                                      flag_list, flag_count, s, qbad, nbad)
    switch (fc_keys(Pe)) {
        case 4: FC_J(4); break;
        case 6: FC_J(6); break;
        default: FC_J(8); break;
    }
#undef FC_J
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
                                                                        int L, int nt, float* __restrict__ D) {
    const int tid = threadIdx.x, lane = tid & 63, g = lane >> 4, c = lane & 15;
    const int h = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int q0 = blockIdx.x * FC_QB;
    u32x4 ah[FC_QBW][DT], al[FC_QBW][DT];
#pragma unroll
    for (int b = 0; b < FC_QBW; b++) {
        const int row_a = q0 + b * 16 + c;
        fc_split_rows<DT>([&](int j) { return row_a < nq ? Q[(size_t)row_a * d + j] : 0.0f; }, d, g, ah[b], al[b]);
    }
    u32x4 bh[2][DT], bl[2][DT];
    fc_prefetch<DT, true>(Cb, nt, h, bh, bl);
    fc_pass<DT, true>(Cb, nt, h, bh, bl, ah, al, [&](const floatx4 (&acc)[FC_QBW], int i, bool) {
        const int col = (FC_NW * i + h) * 16 + c;
#pragma unroll
        for (int b = 0; b < FC_QBW; b++)
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const int row = q0 + b * 16 + 4 * g + r;
                if (row < nq && col < L) D[(size_t)row * L + col] = acc[b][r];
            }
    });
}

void launch_coarse_bf16x3_dots(const float* Q, int nq, int d, const uint4* Cb, int L, float* D,
                               hipStream_t s) {
    if (nq <= 0 || L <= 0) return;
    const int DT = (d + 31) / 32, nt = fc_tiles_per_wave(L);
    const dim3 grid((nq + FC_QB - 1) / FC_QB);
    switch (DT) {
        case 1: hipLaunchKernelGGL(coarse_bf16x3_dots_kernel<1>, grid, dim3(FC_THREADS), 0, s, Q, nq, d, Cb, L, nt, D); break;
        case 2: hipLaunchKernelGGL(coarse_bf16x3_dots_kernel<2>, grid, dim3(FC_THREADS), 0, s, Q, nq, d, Cb, L, nt, D); break;
        case 3: hipLaunchKernelGGL(coarse_bf16x3_dots_kernel<3>, grid, dim3(FC_THREADS), 0, s, Q, nq, d, Cb, L, nt, D); break;
        default: hipLaunchKernelGGL(coarse_bf16x3_dots_kernel<4>, grid, dim3(FC_THREADS), 0, s, Q, nq, d, Cb, L, nt, D); break;
    }
}

}  // namespace vgpu
