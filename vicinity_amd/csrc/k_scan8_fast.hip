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
// Selection.  Each wave keeps its own candidates in its own LDS region:
// entries with fkey(a) <= F (the wave's filter) are appended; when the region
// fills, the wave finds the keep-th smallest key T of its region by ballot
// counts and compacts it to the keys <= T, which become its threshold.  A
// wave's region therefore always holds every entry it scanned with key <= F.
// No barrier is needed until the end of the scan.  T also bounds the query's
// final A_k from above (keep >= k), so every wave may drop entries above
// T + 2 tau: the waves share the smallest such bound.
// At the end, with A_k the k-th smallest approximate distance, the
// reference's top-k lies inside R = {a <= A_k + 2 tau}: the k entries with
// the smallest a have e <= A_k + tau, so the k-th smallest e is at most
// A_k + tau, and any entry of the exact top-k has a <= e + tau <= A_k + 2 tau.
// If the merged regions provably hold R (A_k + 2 tau <= every wave's filter),
// R is rescored with the reference's arithmetic and sorted by (distance,
// insertion index); otherwise a second pass adds the missing keys, and a
// query that still cannot be proved is flagged and rerun by the EXACT kernel.
//
// Layouts.  With codebook_size 256 and 16, 32 or 48 codebooks the lists are
// read from transposed 16-entry blocks (see DevIndex::tcodes), the table is
// stored code-major so that the 16 lanes of a row read 16 different banks,
// and a row's 16 lanes exchange partial sums; otherwise one lane scores one
// list-major code row.
#include <hip/hip_ext.h>

#include "vgpu_device.h"
#include "vgpu_bounds.h"
#include "vgpu_launch.h"

namespace vgpu {

// Native 128-bit vector (raw buffer loads).
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

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

struct FastLds {
    float* lut;      // [M * max(K, 64)] table, then rescoring scratch
    uint64_t* keys;  // [buf] (fkey(a) << 32) | position
    float* qs;       // [d] (prologue only)
    uint32_t* lid;   // [P]
    uint32_t* lbeg;  // [P]
    uint32_t* llen;  // [P]
    uint32_t* pref;  // [P + 1]
    float* term0;    // [P] ||q - c||^2
    // [P] per probed slot, one read per entry: x = lbeg - pref (u32), y = bits
    // of term0; transposed blocks: z = (M + 4) (16 * first block - pref) (u32),
    // w = pref + llen (end of the slot's entries).  In LDS only when P > 64;
    // otherwise lane p holds slot p's record (SlotRegs).
    uint4* bt;
    uint32_t* tbo;   // [P] first transposed block of each probed list
    RadixScratch* rs;
    uint32_t* misc;  // [0] count (merged buffer) [2] lost ties [3..4] second-pass flags by
                     // round parity [5] entries evicted by flushes [6] flushes [7] list
                     // entries probed [8] shared bound on R [9] bits of max ||q - c||^2
                     // [16 + w] wave w's kept count [20 + w] wave w's filter
};

__host__ __device__ inline size_t fs8_align(size_t x) { return (x + 15) & ~(size_t)15; }

// Key buffer: one region per wave, a power of two >= keep + 64 (room for a
// round of appends above the kept keys).
__host__ __device__ inline int fs8_buf(int keep) {
    int b = 1;
    while (b < keep + 64) b <<= 1;
    return b * (VGPU_BLOCK / 64);
}

// Dynamic LDS layout; the table region is omitted when the kernel holds the
// table in a static array (static_lut: compile-time M and K = 256).
__host__ __device__ inline size_t fs8_layout(int d, int M, int K, int P, int buf, bool static_lut,
                                             size_t* off, bool static_rs = false) {
    size_t o = 0;
    const int KL = K > 64 ? K : 64;
    off[0] = o; o = static_lut ? 0 : fs8_align(o + (size_t)M * KL * 4);  // lut
    off[1] = o; o = fs8_align(o + (size_t)buf * 8);        // keys
    off[3] = o; o = fs8_align(o + (size_t)P * 4);          // lid
    off[4] = o; o = fs8_align(o + (size_t)P * 4);          // lbeg
    off[6] = o; o = fs8_align(o + (size_t)(P + 1) * 4);    // pref
    off[8] = o; o = static_rs ? o : fs8_align(o + sizeof(RadixScratch));   // radix scratch
    off[9] = o; o = fs8_align(o + 32 * 4);                 // misc
    off[10] = o; o = fs8_align(o + (P > 64 ? (size_t)P * 16 : 0));  // bt (P <= 64: in registers)
    // qs, llen, term0 and tbo are read only before the scan: they share the
    // key buffer when they fit in it
    const size_t pa = fs8_align((size_t)P * 4), qa = fs8_align((size_t)d * 4);
    if (qa + 3 * pa <= (size_t)buf * 8) {
        off[2] = off[1];
        off[5] = off[1] + qa;
        off[7] = off[5] + pa;
        off[11] = off[7] + pa;
    } else {
        off[2] = o; o += qa;
        off[5] = o; o += pa;
        off[7] = o; o += pa;
        off[11] = o; o += pa;
    }
    return o;
}

__device__ inline FastLds fs8_carve(char* smem, float* static_lut, int d, int M, int K, int P,
                                    int buf, RadixScratch* static_rs = nullptr) {
    size_t off[12];
    fs8_layout(d, M, K, P, buf, static_lut != nullptr, off, static_rs != nullptr);
    FastLds s;
    s.lut = static_lut ? static_lut : (float*)(smem + off[0]);
    s.keys = (uint64_t*)(smem + off[1]);
    s.qs = (float*)(smem + off[2]);
    s.lid = (uint32_t*)(smem + off[3]);
    s.lbeg = (uint32_t*)(smem + off[4]);
    s.llen = (uint32_t*)(smem + off[5]);
    s.pref = (uint32_t*)(smem + off[6]);
    s.term0 = (float*)(smem + off[7]);
    s.rs = static_rs ? static_rs : (RadixScratch*)(smem + off[8]);
    s.misc = (uint32_t*)(smem + off[9]);
    s.bt = (uint4*)(smem + off[10]);
    s.tbo = (uint32_t*)(smem + off[11]);
    return s;
}

// Packed key labels (transposed blocks, P <= 64, fewer than 2^26 padded
// entries per query): the low key word is t | slot << 26, so the probe slot
// and the list position follow without a search over the prefix sums.
#define FS_LBL_BITS 26
#define FS_LBL_MASK ((1u << FS_LBL_BITS) - 1u)

// Block map of the main pass (16 codebooks, transposed blocks, P < 64):
// slot4[b] = 4 x the probe slot of padded block b of the query's
// concatenated lists, vb16[p] = 16 x (the first transposed block of slot p
// less its first padded block), t0[p] = ||q - c||^2 of slot p.  Slot P is a
// sentinel (vb16 0, t0 NaN) for the blocks past the last list, up to the
// last round the main pass reads.  A lane then finds its entry's lane record
// in the transposed blocks and its list term with three LDS reads and one
// add.  The map shares its LDS with
// the radix scratch of the proof, which runs after the main pass; a query
// whose blocks do not fit takes the slot search instead.
#define FS_MAP_BLOCKS 960
struct FsMap {
    uint32_t vb16[65];  // first (the union sits at LDS address 0): vb16 and t0 of a
    float t0[65];       // slot are one paired read at 8-bit dword offsets
    uint8_t slot4[FS_MAP_BLOCKS];
};
union FsAux {
    RadixScratch rs;
    FsMap map;
};
__host__ __device__ constexpr bool fs8_has_map(int MT, int NC) { return NC == 1 && MT == 16; }

// A key (distance, label) as (probe slot << 32) | list position.  Packed
// labels carry the slot; otherwise the largest slot p < P with pref[p] <= t
// is the non-empty list holding t.
__device__ __forceinline__ uint64_t fs8_relabel(const FastLds& s, uint64_t v, int P, bool packed) {
    const uint32_t lo32 = (uint32_t)v;
    if (packed) {
        const uint32_t p = lo32 >> FS_LBL_BITS;
        return ((uint64_t)p << 32) | (s.lbeg[p] - s.pref[p] + (lo32 & FS_LBL_MASK));
    }
    uint32_t lo = 0, hi = (uint32_t)P;
    while (hi - lo > 1u) {
        const uint32_t mid = (lo + hi) >> 1;
        if (s.pref[mid] <= lo32) lo = mid;
        else hi = mid;
    }
    return ((uint64_t)lo << 32) | (s.lbeg[lo] + (lo32 - s.pref[lo]));
}

// Keep the keys key_at(0 .. n) whose high word is <= T, written densely to
// keys[0 ..) chunk by chunk: a chunk is read into registers before any slot
// is rewritten, and the compacted prefix never passes the slot of a key not
// yet read (key_at(i) is stored at or after keys[i]).  Keys carry t, the
// entry's index in the concatenated probed lists; with `relabel`, each kept
// key is rewritten as (probe slot << 32) | position, the slot found by binary
// search over the list prefix sums.
template <typename KeyAt>
__device__ inline uint32_t fs8_compact(FastLds& s, KeyAt key_at, uint32_t n, uint32_t T, bool relabel,
                                       int P, bool packed) {
    const int tid = threadIdx.x;
    __syncthreads();
    if (tid == 0) s.misc[0] = 0;
    __syncthreads();
    for (uint32_t c0 = 0; c0 < n; c0 += VGPU_BLOCK) {
        const uint32_t i = c0 + tid;
        uint64_t v = i < n ? key_at(i) : ~0ull;
        bool take = i < n && (uint32_t)(v >> 32) <= T;
        __syncthreads();
        if (take && relabel) v = fs8_relabel(s, v, P, packed);
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
template <typename KeyAt>
__device__ uint32_t fs8_select_upper(FastLds& s, KeyAt key_at, uint32_t n, uint32_t rank, uint32_t limit) {
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    uint32_t mn = 0xffffffffu, mx = 0u;
    for (uint32_t i = tid; i < n; i += VGPU_BLOCK) {
        const uint32_t h = (uint32_t)(key_at(i) >> 32);
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
        atomicAdd(&s.rs->hist[((uint32_t)(key_at(i) >> 32) >> shift) & 255u], 1u);
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
        auto hk = [&](int i) -> uint32_t { return (uint32_t)(key_at((uint32_t)i) >> 32); };
        return block_radix_select<uint32_t>(hk, (int)n, rank, s.rs);
    }
    const uint32_t low = (1u << shift) - 1u;
    const uint32_t base = sbit >= 31 ? 0u : (mn & ~((2u << sbit) - 1u));  // common prefix
    return base | (b << shift) | low;
}

// Per-thread state of the entries one thread handles in one round.  The
// loads are unconditional (a slot past the end reads position 0, which exists
// whenever anything is scanned) so the compiler can wait for one round's
// loads while the next rounds' are still in flight.
template <int MT>
struct RoundRegs {
    CodeRow<MT> row[FS_U];
    float bias[FS_U];
    float t0[FS_U];    // ||q - c||^2 of the entry's list; NaN: no entry (past a list's end)
    uint32_t pos[FS_U];// position (code row), generic path only
    uint32_t t[FS_U];  // index in the concatenated probed lists
};

// Slot records of the probed lists held in lane registers when P <= 64:
// lane p holds pref[p] (0xffffffff for p >= P) and bt[p].
struct SlotRegs {
    uint32_t pref;
    uint4 bt;
};

__device__ __forceinline__ uint4 readlane4(const uint4& v, int lane) {
    return make_uint4(__builtin_amdgcn_readlane(v.x, lane), __builtin_amdgcn_readlane(v.y, lane),
                      __builtin_amdgcn_readlane(v.z, lane), __builtin_amdgcn_readlane(v.w, lane));
}

// Record of the probed slot holding index x of the window [wb, wb + 64): the
// last slot p with pref[p] <= x (empty lists repeat a start and are passed
// over).  With P <= 64 it comes from the lane registers: the slot of the
// window start is a ballot count, then each list start inside the window
// (usually none or one) is read out and the lanes at or past it switch to its
// record.  Otherwise the wave keeps a cursor cw over the LDS prefix sums
// (windows only move forward) and counts the starts inside the window.
// *slot (when given) receives the slot index.
__device__ __forceinline__ uint4 slot_record(const FastLds& s, const SlotRegs& r, int P, uint32_t wb,
                                             uint32_t x, int& cw, uint32_t* slot = nullptr) {
    if (P <= 64) {
        const int c = (int)__popcll(__ballot(r.pref <= wb)) - 1;
        uint4 e = readlane4(r.bt, c);
        uint32_t sl = (uint32_t)c;
        uint64_t inwin = __ballot(r.pref > wb && r.pref < wb + 64u);
        while (inwin) {
            const int p = (int)__builtin_ctzll(inwin);
            inwin &= inwin - 1;
            const uint32_t b = __builtin_amdgcn_readlane(r.pref, p);
            const uint4 f = readlane4(r.bt, p);
            if (x >= b) {
                e = f;
                sl = (uint32_t)p;
            }
        }
        if (slot) *slot = sl;
        return e;
    }
    while (cw + 1 < P && __builtin_amdgcn_readfirstlane(s.pref[cw + 1]) <= wb) cw++;
    int lst = cw;
    for (int j = cw + 1; j < P; j++) {
        const uint32_t b = __builtin_amdgcn_readfirstlane(s.pref[j]);
        if (b >= wb + 64u) break;
        lst += x >= b ? 1 : 0;
    }
    if (slot) *slot = (uint32_t)lst;
    return s.bt[lst];
}


// Entry t = rbase + wave * 64 + lane: the waves take interleaved windows of
// 64 consecutive entries.
template <int MT>
__device__ __forceinline__ void fs8_fetch(const DevIndex& ix, const FastLds& s, const SlotRegs& sr,
                                          uint32_t rbase, uint32_t total, int P, int& cw,
                                          RoundRegs<MT>& g) {
    static_assert(FS_U == 1, "one window per wave and round");
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    {
        constexpr int u = 0;
        const uint32_t wb = rbase + wave * 64u;  // window start
        const uint32_t t = wb + lane;
        const bool valid = t < total;
        const uint4 e = slot_record(s, sr, P, wb, t, cw);
        const uint32_t pos = valid ? e.x + t : 0u;
        g.pos[u] = pos;
        g.t[u] = t;
        g.t0[u] = valid ? __uint_as_float(e.y) : __builtin_nanf("");
        if constexpr (MT > 0) load_row<MT>(g.row[u], ix.codes + (size_t)pos * MT);
        g.bias[u] = ix.bias[pos];
    }
}

// Structured buffer loads (index x stride + offset, range-checked by index,
// zeros past the last record): the LLVM intrinsics, which have no clang
// builtin.
__device__ u32x4 fs8_sload4(__amdgpu_buffer_rsrc_t rsrc, uint32_t vindex, uint32_t voffset, uint32_t soffset,
                            int aux) __asm("llvm.amdgcn.struct.ptr.buffer.load.v4i32");
__device__ uint32_t fs8_sload1(__amdgpu_buffer_rsrc_t rsrc, uint32_t vindex, uint32_t voffset, uint32_t soffset,
                               int aux) __asm("llvm.amdgcn.struct.ptr.buffer.load.i32");

// The codes and b(x) of lane record `vi` of the transposed blocks: `rsc`
// addresses tcodes in records of MT bytes, `rsb` tbias in records of one
// float, so both loads take the one index register and no offset.
template <int MT>
__device__ __forceinline__ void fs8t_load(__amdgpu_buffer_rsrc_t rsc, __amdgpu_buffer_rsrc_t rsb, uint32_t vi,
                                          RoundRegs<MT>& g) {
#pragma unroll
    for (int gi = 0; gi < MT / 16; gi++) {
        const u32x4 x = fs8_sload4(rsc, vi, 16u * gi, 0u, 0);
        g.row[0].w[4 * gi] = x.x;
        g.row[0].w[4 * gi + 1] = x.y;
        g.row[0].w[4 * gi + 2] = x.z;
        g.row[0].w[4 * gi + 3] = x.w;
    }
    g.bias[0] = __uint_as_float(fs8_sload1(rsb, vi, 0u, 0u, 0));
}

// Transposed blocks: the probed lists are concatenated in whole 16-entry
// blocks (t runs over the padded sequence, pref holds padded starts).  A
// wave's window of 64 entries is four blocks, one per row of 16 lanes; lane
// (row, m) loads lane record m of its row's block: the 16 codes of codebooks
// m, m + 16, ... (code j of entry j ^ m) and the b(x) of the block's entry
// m, which is the entry it ends up scoring.  The record index is the slot's
// e.z = 16 x its first block - pref, plus t; rows past the end of the lists
// read zeros or an unrelated record, and their entries are invalid (NaN
// term).
template <int MT>
__device__ __forceinline__ void fs8t_fetch(__amdgpu_buffer_rsrc_t rsc, __amdgpu_buffer_rsrc_t rsb, const FastLds& s,
                                           const SlotRegs& sr, uint32_t rbase, int P, int& cw, RoundRegs<MT>& g,
                                           bool packed) {
    static_assert(FS_U == 1 && MT % 16 == 0, "one window per wave and round");
    const uint32_t lane = threadIdx.x & 63u, m = lane & 15u;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t wb = rbase + wave * 64u;  // window start
    const uint32_t tb = wb + (lane & 48u);   // the row's block start
    const uint32_t t = tb + m;
    uint32_t base;  // record index of the window's first entry (the lane adds its own)
    float t0;
    uint32_t slot = 0;
    bool uniform = false;
    if (P <= 64) {
        // Usually one list covers the whole window (no list starts inside it
        // and none ends before its last entry): its record is read into
        // scalars once and the lanes share it.
        const uint64_t le = __ballot(sr.pref <= wb), lt = __ballot(sr.pref < wb + 64u);
        const int c = (int)__popcll(le) - 1;
        const uint32_t ez = __builtin_amdgcn_readlane(sr.bt.z, c), ey = __builtin_amdgcn_readlane(sr.bt.y, c);
        const uint32_t ew = __builtin_amdgcn_readlane(sr.bt.w, c);
        if (lt == le && ew >= wb + 64u) {
            uniform = true;
            base = ez + wb;
            t0 = __uint_as_float(ey);
            slot = (uint32_t)c;
        }
    }
    if (!uniform) {
        const uint4 e = slot_record(s, sr, P, wb, tb, cw, &slot);
        base = e.z + wb;
        t0 = t < e.w ? __uint_as_float(e.y) : __builtin_nanf("");
    }
    fs8t_load<MT>(rsc, rsb, base + lane, g);
    g.t0[0] = t0;
    g.t[0] = packed ? t | slot << FS_LBL_BITS : t;
}

// Main-pass fetch through the block map, in three stages one round apart so
// that no stage waits on the LDS read of another: the map byte of round
// f + 2, the record of round f + 1 from its map byte, and the loads of round
// f from its record.  Lane (row, m) of the window at wb scores entry m of
// padded block wb / 16 + row, whose lane record is 16 vb[slot] + wb + lane,
// so the record index is one add.  A sentinel row reads record wb + lane (or
// zeros past the end) and its NaN t0 keeps its entries out.  Labels are
// packed.
struct MapPipe {
    uint32_t s4n;  // map byte of the round after next
    uint32_t vi;   // next round: lane record, packed label, t0
    uint32_t lbl;
    float t0;
};

__device__ __forceinline__ uint32_t fs8m_byte(const FsMap& mp, uint32_t rbase) {
    const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t b0 = __builtin_amdgcn_readfirstlane((rbase + wave * 64u) >> 4);  // the window's first block
    return mp.slot4[b0 + ((threadIdx.x & 63u) >> 4)];
}

__device__ __forceinline__ void fs8m_record(const FsMap& mp, uint32_t rbase, uint32_t s4, MapPipe& mpp) {
    const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t t = rbase + wave * 64u + (threadIdx.x & 63u);  // wb + lane
    mpp.vi = *reinterpret_cast<const uint32_t*>(reinterpret_cast<const char*>(mp.vb16) + s4) + t;
    mpp.t0 = *reinterpret_cast<const float*>(reinterpret_cast<const char*>(mp.t0) + s4);
    mpp.lbl = t | (s4 << (FS_LBL_BITS - 2));
}

template <int MT>
__device__ __forceinline__ void fs8m_fetch(__amdgpu_buffer_rsrc_t rsc, __amdgpu_buffer_rsrc_t rsb, const FsMap& mp,
                                           uint32_t rbase, MapPipe& mpp, RoundRegs<MT>& g) {
    static_assert(FS_U == 1 && MT % 16 == 0, "one window per wave and round");
    fs8t_load<MT>(rsc, rsb, mpp.vi, g);
    g.t0[0] = mpp.t0;
    g.t[0] = mpp.lbl;
    fs8m_record(mp, rbase + FS_ROUND, mpp.s4n, mpp);
    mpp.s4n = fs8m_byte(mp, rbase + 2 * FS_ROUND);
}

// a + DPP-moved b (row-local patterns, every source lane active, so no lane
// takes the bound_ctrl zero; the move folds into the add).
template <int CTRL>
__device__ __forceinline__ float add_dpp(float a, float b) {
    return a + __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(b), CTRL, 0xF, 0xF, true));
}

// Transposed table: T2[m][c] of codebook m = 16 gi + r lives at float
// ((gi * 256 + c) * NC + copy) * 16 + r, in NC copies; the lanes of row w read
// copy w % NC, so a half wave (two rows) reads 32 distinct banks when NC = 2.
// `lutl` is the table plus the lane's (copy * 16 + m).  Lane m's terms v[j]
// belong to entry j ^ m of its row; four exchange stages with the lanes m ^ 1,
// m ^ 2, m ^ 7 and m ^ 8 (each halving the registers still needed) leave the
// sum of entry m in v[0].  Every lane of the wave must be active.
// c * 64 + off for the code c held in the low (HI = 0) or high (HI = 1)
// 16-bit half of h (the other half is ignored): one v_mad_u32_u16 with op_sel.
template <int HI>
__device__ __forceinline__ uint32_t code_addr(uint32_t h, uint32_t off) {
    uint32_t a;
    if constexpr (HI) asm("v_mad_u32_u16 %0, %1, 64, %2 op_sel:[1,0,0,0]" : "=v"(a) : "v"(h), "v"(off));
    else asm("v_mad_u32_u16 %0, %1, 64, %2" : "=v"(a) : "v"(h), "v"(off));
    return a;
}

template <int MT, int NC>
__device__ __forceinline__ float trow_sum(const CodeRow<MT>& r, const float* __restrict__ lutl) {
    float v[16];
    if constexpr (NC == 1) {
        // Byte offsets c * 64 + 4 m: codes 0 and 2 of a word are split into
        // 16-bit halves by a mask, codes 1 and 3 by a byte permute, and each
        // offset is one multiply-add on a half (1.5 instructions per code).
        const float* lut0 = lutl - (threadIdx.x & 15);
        const uint32_t m4 = (threadIdx.x & 15u) * 4u;
#pragma unroll
        for (int gi = 0; gi < MT / 16; gi++) {
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const uint32_t w = r.w[4 * gi + i];
                const uint32_t h02 = w & 0x00ff00ffu;                       // codes 0, 2
                const uint32_t h13 = __builtin_amdgcn_perm(0u, w, 0x0c030c01u);  // codes 1, 3
                const uint32_t o[4] = {code_addr<0>(h02, m4), code_addr<0>(h13, m4), code_addr<1>(h02, m4),
                                       code_addr<1>(h13, m4)};
#pragma unroll
                for (int b = 0; b < 4; b++) {
                    const float x = *reinterpret_cast<const float*>(
                        reinterpret_cast<const char*>(lut0 + gi * 256 * 16) + o[b]);
                    v[4 * i + b] = gi == 0 ? x : v[4 * i + b] + x;
                }
            }
        }
    } else {
#pragma unroll
        for (int j = 0; j < 16; j++) {
#pragma unroll
            for (int gi = 0; gi < MT / 16; gi++) {
                const uint32_t c = (r.w[4 * gi + (j >> 2)] >> (8 * (j & 3))) & 0xffu;
                const float x = lutl[(gi * 256 + (int)c) * NC * 16];
                v[j] = gi == 0 ? x : v[j] + x;
            }
        }
    }
#pragma unroll
    for (int j = 0; j < 16; j++)  // keep 0 2 5 7 8 10 13 15 (partner m ^ 1)
        if (j == 0 || j == 2 || j == 5 || j == 7 || j == 8 || j == 10 || j == 13 || j == 15)
            v[j] = add_dpp<0xB1>(v[j], v[j ^ 1]);
    v[0] = add_dpp<0x4E>(v[0], v[2]);   // partner m ^ 2
    v[7] = add_dpp<0x4E>(v[7], v[5]);
    v[8] = add_dpp<0x4E>(v[8], v[10]);
    v[15] = add_dpp<0x4E>(v[15], v[13]);
    v[0] = add_dpp<0x141>(v[0], v[7]);  // partner m ^ 7 (row_half_mirror)
    v[8] = add_dpp<0x141>(v[8], v[15]);
    return add_dpp<0x128>(v[0], v[8]);  // partner m ^ 8 (row_ror:8)
}

// Approximate distance a of the entry a lane holds in g (every lane of the
// wave must take part: the transposed sum exchanges values between lanes).
template <int MT, int KT, int NC>
__device__ __forceinline__ float entry_dist(const DevIndex& ix, const FastLds& s, const float* lut_static,
                                            const RoundRegs<MT>& g) {
    const int lane = threadIdx.x & 63;
    if constexpr (NC > 0) {
        const float* lutl = lut_static + (((lane >> 4) & (NC - 1)) * 16 + (lane & 15));
        return (g.t0[0] + g.bias[0]) + trow_sum<MT, NC>(g.row[0], lutl);
    } else if constexpr (MT > 0 && KT > 0) {
        return (g.t0[0] + g.bias[0]) + row_sum<MT, KT>(g.row[0], lut_static);
    } else {
        return (g.t0[0] + g.bias[0]) + row_sum_generic(ix.codes + (size_t)g.pos[0] * ix.M, s.lut, ix.M, ix.K);
    }
}

// Main pass: append the entries with fkey(a) <= F to the wave's own region
// `reg` (no atomics: the count is the wave's own).  The region has room for
// a round (cnt <= capacity - 64 on entry).
template <int MT, int KT, int NC>
__device__ __forceinline__ void fs8w_consume(const DevIndex& ix, const FastLds& s, const float* lut_static,
                                             const RoundRegs<MT>& g, float Ff, uint64_t* reg,
                                             uint32_t& cnt) {
    const float dist = entry_dist<MT, KT, NC>(ix, s, lut_static, g);
    const bool take = dist <= Ff;  // NaN (no entry) never
    const uint64_t mask = __ballot(take);
    if (mask == 0) return;  // wave-uniform
    if (take) {
        const uint32_t below =
            __builtin_amdgcn_mbcnt_hi((uint32_t)(mask >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)mask, 0u));
        reg[cnt + below] = ((uint64_t)fkey(dist) << 32) | g.t[0];
    }
    cnt += (uint32_t)__popcll(mask);
}

// The float threshold equivalent to a key filter F on the approximate
// distances: x <= filter_float(F) exactly when fkey(x) <= F, for finite x
// other than -0.0 (an approximate distance is (t0 + b(x)) + sum with
// t0 = ||q - c||^2 >= +0, so it is never -0.0).
__device__ __forceinline__ float filter_float(uint32_t F) {
    uint32_t b = (F & 0x80000000u) ? (F & 0x7fffffffu) : ~F;  // fkey_to_float
    b = F >= 0xff800000u ? 0x7f800000u : b;                   // every finite distance
    b = F == 0x7fffffffu ? 0x80000001u : b;                   // the negative ones
    return __uint_as_float(__builtin_amdgcn_readfirstlane(b));  // wave-uniform
}

// Second pass (after the regions are merged into one buffer): append the keys
// in (lo, hi] with one LDS atomic per wave.  A wave whose appends took the
// buffer past `cap` raises flag misc[3 + parity] (the parities alternate
// between rounds; the caller reads the flag after a barrier).
template <int MT, int KT, int NC>
__device__ __forceinline__ void fs8_consume_retry(const DevIndex& ix, FastLds& s, const float* lut_static,
                                                  const RoundRegs<MT>& g, uint32_t hi, uint32_t lo,
                                                  uint32_t cap, int parity) {
    const int lane = threadIdx.x & 63;
    const float dist = entry_dist<MT, KT, NC>(ix, s, lut_static, g);
    const uint32_t fk = fkey(dist);
    const bool take = dist == dist && fk <= hi && fk > lo;  // NaN: no entry
    const uint64_t mask = __ballot(take);
    const uint32_t tot = (uint32_t)__popcll(mask);
    if (tot == 0) return;  // wave-uniform
    uint32_t base = 0;
    if (lane == 0) base = atomicAdd(&s.misc[0], tot);
    base = __builtin_amdgcn_readfirstlane(base);
    if (take) {
        const uint32_t below =
            __builtin_amdgcn_mbcnt_hi((uint32_t)(mask >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)mask, 0u));
        s.keys[base + below] = ((uint64_t)fk << 32) | g.t[0];
    }
    if (base + tot > cap && lane == 0) s.misc[3 + parity] = 1u;
}

// Wave-level flush of the wave's region reg[0, cnt): T = the rank-th smallest
// high word (0-based), found bit by bit from the top with ballot counts; the
// search stops early once every key up to the top of T's current prefix
// range fits `capw` (T is then that upper end).  The keys <= T are compacted
// in place (each chunk of 64 is read before any of its slots is rewritten).
// Returns T; cnt becomes the kept count, or capw with *lost set when more
// than capw keys are <= T (ties).
__device__ uint32_t fs8w_flush(uint64_t* reg, uint32_t& cnt, uint32_t rank, uint32_t capw, bool* lost) {
    const uint32_t lane = threadIdx.x & 63u;
    uint32_t h[4];
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const uint32_t idx = (uint32_t)i * 64u + lane;
        h[i] = idx < cnt ? (uint32_t)(reg[idx] >> 32) : 0xffffffffu;
    }
    // keys (high words) < v, counting the ones past the first 256 from LDS
    auto below = [&](uint32_t v) -> uint32_t {
        uint32_t c = 0;
#pragma unroll
        for (int i = 0; i < 4; i++) c += (uint32_t)__popcll(__ballot(h[i] < v));
        for (uint32_t i0 = 256; i0 < cnt; i0 += 64) {
            const uint32_t idx = i0 + lane;
            const uint32_t x = idx < cnt ? (uint32_t)(reg[idx] >> 32) : 0xffffffffu;
            c += (uint32_t)__popcll(__ballot(x < v));
        }
        return c;
    };
    uint32_t T = 0;
    for (int b = 31; b >= 0; b--) {
        const uint32_t cand = T | (1u << b);
        if (below(cand) <= rank) T = cand;
        if ((b & 3) == 0 && b > 0) {  // T's prefix is final down to bit b
            const uint32_t top = T | ((1u << b) - 1u);
            if (top != 0xffffffffu && below(top + 1u) <= capw) {
                T = top;
                break;
            }
        }
    }
    uint32_t kept = 0;
    for (uint32_t i0 = 0; i0 < cnt; i0 += 64) {
        const uint32_t idx = i0 + lane;
        const uint64_t v = idx < cnt ? reg[idx] : ~0ull;
        const bool take = idx < cnt && (uint32_t)(v >> 32) <= T;
        const uint64_t mask = __ballot(take);
        if (take) {
            const uint32_t at = kept + __builtin_amdgcn_mbcnt_hi((uint32_t)(mask >> 32),
                                                                  __builtin_amdgcn_mbcnt_lo((uint32_t)mask, 0u));
            if (at < capw) reg[at] = v;
        }
        kept += (uint32_t)__popcll(mask);
    }
    if (kept > capw) {
        *lost = true;
        kept = capw;
    }
    cnt = kept;
    return T;
}

// Dense index i of the merged regions -> LDS slot (region w holds cw[w]
// keys at w * BW).
__device__ __forceinline__ uint32_t region_slot(uint32_t i, const uint32_t* off, uint32_t BW) {
    uint32_t w = 0;
#pragma unroll
    for (int v = 1; v < VGPU_BLOCK / 64; v++) w += i >= off[v] ? 1u : 0u;
    return w * BW + (i - off[w]);
}

// Merge the waves' regions into keys[0, n) (dense order, chunk by chunk: a
// slot is rewritten only after every key stored at or before it was read,
// because region w starts at w * BW >= the keys of the regions before it).
__device__ inline uint32_t fs8w_merge(FastLds& s, const uint32_t* cnts, uint32_t BW) {
    uint32_t off[VGPU_BLOCK / 64 + 1];
    off[0] = 0;
#pragma unroll
    for (int w = 0; w < VGPU_BLOCK / 64; w++) off[w + 1] = off[w] + cnts[w];
    const uint32_t n = off[VGPU_BLOCK / 64];
    for (uint32_t c0 = 0; c0 < n; c0 += VGPU_BLOCK) {
        const uint32_t i = c0 + threadIdx.x;
        const uint64_t v = i < n ? s.keys[region_slot(i, off, BW)] : 0ull;
        __syncthreads();
        if (i < n) s.keys[i] = v;
        __syncthreads();
    }
    return n;
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
// (0 = read from the index at run time).  NC > 0: the lists are read from the
// transposed blocks, with NC copies of the table.
// Exact distance (the reference's arithmetic, pq_simd.rs:349-355) of the list
// entry whose code row both lanes half = 0, 1 of a pair hold: lane `half`
// takes codebooks M/2 half .. (or, DS = 8, codebooks 2t + half, at most TBW
// codewords' loads in flight), with the residual r = q - c of the entry's
// probe slot p at res + p * D (LDS); the first lane adds the sub-distances in
// codebook order from 0.0 and continues with its partner's, handed over by a
// lane exchange, and returns the distance (the second lane's return value is
// unused).  Both lanes of every pair must take part.
template <int MT, int KT, int DS, int TBW>
__device__ __forceinline__ float fs8_pair_distance(const DevIndex& ix, const float* __restrict__ res,
                                                   uint32_t p, const CodeRow<MT>& row, uint32_t half) {
    constexpr int D = MT * DS;
    constexpr int H = MT / 2;                 // codebooks per thread
    constexpr int CB1 = 64 / DS < H ? 64 / DS : H;
    constexpr int CB = CB1 >= 16 ? 16 : CB1 >= 8 ? 8 : CB1 >= 4 ? 4 : CB1 >= 2 ? 2 : 1;  // codewords in flight
    static_assert(H % CB == 0 && H % 4 == 0, "codebook batches");
    constexpr int HW = H / 4;                 // code words per half row
    uint32_t cwd[HW];
#pragma unroll
    for (int w = 0; w < HW; w++) cwd[w] = half ? row.w[HW + w] : row.w[w];  // no dynamic register index
    float total_e = 0.0f;
    if constexpr (DS == 8) {
        // The pair shares its codewords: for codebooks 2t and 2t + 1 lane
        // `half` loads dims 4 half .. 4 half + 3 of both (the two lanes of a
        // load read one codeword, one cache access), gives its partner the
        // half it lacks (lane 0 scores 2t, lane 1 scores 2t + 1) and takes its
        // residual slice from LDS; lane 0 then adds the scores in codebook
        // order.  Raw buffer loads at 32-bit offsets.
        const __amdgpu_buffer_rsrc_t cbr = __builtin_amdgcn_make_buffer_rsrc(
            const_cast<float*>(ix.codebooks), (short)0, MT * KT * DS * 4, 0x00020000);
        float ev[MT / 2];  // this lane's codebooks 2t + half
        const float* rrow = res + (size_t)p * D + half * DS;
        const uint32_t hoff = half * 16u;
        constexpr int TB = MT / 2 < TBW ? MT / 2 : TBW;  // codebook pairs whose loads fly together
#pragma unroll
        for (int t0 = 0; t0 < MT / 2; t0 += TB) {
            u32x4 Ab[TB], Bb[TB];
#pragma unroll
            for (int tb = 0; tb < TB; tb++) {  // every load of the batch first
                const int t = t0 + tb;
                const uint32_t w = row.w[t >> 1];
                const uint32_t c0 = (w >> (16 * (t & 1))) & 0xffu, c1 = (w >> (16 * (t & 1) + 8)) & 0xffu;
                Ab[tb] = __builtin_amdgcn_raw_buffer_load_b128(
                    cbr, c0 * (uint32_t)(DS * 4) + hoff + (uint32_t)(2 * t * KT * DS * 4), 0u, 0);
                Bb[tb] = __builtin_amdgcn_raw_buffer_load_b128(
                    cbr, c1 * (uint32_t)(DS * 4) + hoff + (uint32_t)((2 * t + 1) * KT * DS * 4), 0u, 0);
            }
#pragma unroll
            for (int tb = 0; tb < TB; tb++) {
                const int t = t0 + tb;
                const u32x4 A = Ab[tb], B = Bb[tb];
                const u32x4 snd = half ? A : B;
                u32x4 rcv;
                rcv.x = (uint32_t)__builtin_amdgcn_mov_dpp((int)snd.x, 0xB1, 0xF, 0xF, true);
                rcv.y = (uint32_t)__builtin_amdgcn_mov_dpp((int)snd.y, 0xB1, 0xF, 0xF, true);
                rcv.z = (uint32_t)__builtin_amdgcn_mov_dpp((int)snd.z, 0xB1, 0xF, 0xF, true);
                rcv.w = (uint32_t)__builtin_amdgcn_mov_dpp((int)snd.w, 0xB1, 0xF, 0xF, true);
                const u32x4 lo = half ? rcv : A, hi = half ? B : rcv;
                const float cw[8] = {__uint_as_float(lo.x), __uint_as_float(lo.y), __uint_as_float(lo.z),
                                     __uint_as_float(lo.w), __uint_as_float(hi.x), __uint_as_float(hi.y),
                                     __uint_as_float(hi.z), __uint_as_float(hi.w)};
                const float* r = rrow + (size_t)(2 * t) * DS;  // codebook 2t + half
                float e = 0.0f;
#pragma unroll
                for (int j = 0; j < 8; j++) {
                    const float diff = __fsub_rn(r[j], cw[j]);
                    e = __fadd_rn(e, __fmul_rn(diff, diff));
                }
                ev[t] = e;
            }
        }
#pragma unroll
        for (int t = 0; t < MT / 2; t++) {  // lane 0: e_2t, then the partner's e_2t+1
            total_e = __fadd_rn(total_e, ev[t]);
            total_e = __fadd_rn(total_e, __int_as_float(__builtin_amdgcn_mov_dpp(
                                             __float_as_int(ev[t]), 0xB1, 0xF, 0xF, true)));
        }
    } else {
    float ev[H];
    const float* rrow = res + (size_t)p * D + half * H * DS;
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
    // codebooks 0 .. H - 1 (first thread)
#pragma unroll
    for (int h = 0; h < H; h++) total_e = __fadd_rn(total_e, ev[h]);
#pragma unroll
    for (int h = 0; h < H; h++)  // then the partner's H .. M - 1
        total_e = __fadd_rn(total_e, __uint_as_float(shfl_xor_u32(__float_as_uint(ev[h]), 1)));
    }
    return total_e;
}

// PRE: the per-query table T2 was written by t2_table_kernel (a.t2) and is
// copied into LDS instead of being built here.
template <int MT, int KT, int DS, int NC, int PRE>
__global__ __launch_bounds__(256, 6) void scan8_fast_kernel(DevIndex ix, ScanArgs a, int buf) {
    constexpr bool TR = NC > 0;
    static_assert(!TR || (MT % 16 == 0 && KT == 256 && DS > 0), "transposed blocks");
    static_assert(!PRE || (TR && NC == 1), "precomputed tables: transposed layout, one copy");
    constexpr bool kStatic = MT > 0 && KT >= 64;
    constexpr int D = MT * DS;  // compile-time dimension when > 0
    constexpr int LUTF = kStatic ? MT * KT * (TR ? NC : 1) : 1;  // static table floats
    constexpr bool kMap = fs8_has_map(MT, NC);
    // Static LDS: the block map / radix scratch (kMap) at address 0, then the table.
    constexpr int AUXB = kMap ? (int)((sizeof(FsAux) + 15) & ~(size_t)15) : 0;
    __shared__ __align__(16) char sstat[AUXB + LUTF * 4];
    float* const slut = reinterpret_cast<float*>(sstat + AUXB);
    extern __shared__ __align__(16) char smem[];
    const int q = blockIdx.x;
    if (q >= a.nq) return;
    const int tid = threadIdx.x, lane = tid & 63;
    const int d = D > 0 ? D : ix.d, M = MT > 0 ? MT : ix.M, K = KT > 0 ? KT : ix.K;
    const int ds = DS > 0 ? DS : ix.ds, P = a.P;
    FsAux* aux = reinterpret_cast<FsAux*>(sstat);
    FastLds s = fs8_carve(smem, kStatic ? slut : nullptr, d, M, K, P, buf, kMap ? &aux->rs : nullptr);

    // ---- prologue: query, probed lists, ||q - c||^2, the per-query table.
    // Round trip 1: the thread's first probed slot and (blocks) the query
    // slices and first codebook lines of the table; round trip 2: that slot's
    // list record with the next codebook lines.  Slots past the first 256 are
    // read afterwards.
    const uint32_t l0id = tid < P ? a.probe[(size_t)q * P + tid] : 0u;
    // a probed slot's list record (list, begin, end, block offset): loads,
    // then (once they are back) LDS stores
    uint32_t rl = 0, rb = 0, re = 0, rt = 0;
    auto rec_load = [&](uint32_t l) {
        const bool ok = l < (uint32_t)ix.L;  // no such list: scanned as empty
        rl = ok ? l : 0u;
        rb = ok ? ix.offsets[l] : 0u;
        re = ok ? ix.offsets[l + 1] : 0u;
        if constexpr (TR) rt = ok ? ix.tblk_off[l] : 0u;
    };
    auto rec_store = [&](int p) {
        s.lid[p] = rl;
        s.lbeg[p] = rb;
        s.llen[p] = re - rb;
        if constexpr (TR) s.tbo[p] = rt;
    };
    if (tid < 32) s.misc[tid] = tid == 8 ? 0xffffffffu : 0u;  // counts 0, no bound yet
    // PRE: eight lanes per probed slot (the first PG slots) form ||q - c||^2
    // of their slot here.  The residual itself is not held until the
    // rescoring: sixteen more registers across the main pass spilled 32 bytes
    // per lane to scratch (70 MB of writes per 10k batch); the rescoring
    // stages it again from the centroids.
    constexpr int PG = VGPU_BLOCK / 8;
    if constexpr (PRE) {
        // Two round trips.  First: the query's table (LUTF floats, coalesced
        // 16-byte pieces), the query, the thread's probed slot and the slot of
        // its eight-lane group.  Second: the slot's list record and the group
        // slot's centroid slices, from which ||q - c||^2 follows.
        constexpr int TPT = LUTF / 4 / VGPU_BLOCK;  // 16-byte pieces per thread
        static_assert(LUTF % (4 * VGPU_BLOCK) == 0 && D % 32 == 0 && D / 4 <= VGPU_BLOCK, "table copy split");
        const float4* src = reinterpret_cast<const float4*>(a.t2 + (size_t)q * LUTF);
        float4 tv[TPT];
#pragma unroll
        for (int i = 0; i < TPT; i++) tv[i] = src[i * VGPU_BLOCK + tid];
        const int g = tid >> 3, sub = tid & 7;
        const uint32_t gid = g < P ? a.probe[(size_t)q * P + g] : 0u;
        const float4* qrow = reinterpret_cast<const float4*>(a.qn + (size_t)q * D);
        float4 qsl[D / 32];
#pragma unroll
        for (int i = 0; i < D / 32; i++) qsl[i] = qrow[8 * i + sub];
        // the table is stored before the second round trip is issued (that
        // round trip waits on the probed ids anyway), which frees its registers
        float4* dst = reinterpret_cast<float4*>(slut);
#pragma unroll
        for (int i = 0; i < TPT; i++) dst[i * VGPU_BLOCK + tid] = tv[i];
        if (tid < P) rec_load(l0id);
        const bool gok = g < P && gid < (uint32_t)ix.L;  // no such list: scanned as empty
        const float4* crow = reinterpret_cast<const float4*>(ix.centroids + (size_t)(gok ? gid : 0u) * D);
        float4 cv[D / 32];
#pragma unroll
        for (int i = 0; i < D / 32; i++) cv[i] = crow[8 * i + sub];
        if (g == 0) {  // the query itself: group 0's lanes hold every dimension once
#pragma unroll
            for (int i = 0; i < D / 32; i++) reinterpret_cast<float4*>(s.qs)[8 * i + sub] = qsl[i];
        }
        if (tid < P) rec_store(tid);
        float acc = 0.0f;  // ||q - c||^2, ranking only: any order, FMA allowed
#pragma unroll
        for (int i = 0; i < D / 32; i++) {
            const float4 r = make_float4(__fsub_rn(qsl[i].x, cv[i].x), __fsub_rn(qsl[i].y, cv[i].y),
                                         __fsub_rn(qsl[i].z, cv[i].z), __fsub_rn(qsl[i].w, cv[i].w));
            acc = __builtin_fmaf(r.x, r.x, acc);
            acc = __builtin_fmaf(r.y, r.y, acc);
            acc = __builtin_fmaf(r.z, r.z, acc);
            acc = __builtin_fmaf(r.w, r.w, acc);
        }
        acc += __uint_as_float(shfl_xor_u32(__float_as_uint(acc), 1));
        acc += __uint_as_float(shfl_xor_u32(__float_as_uint(acc), 2));
        acc += __uint_as_float(shfl_xor_u32(__float_as_uint(acc), 4));
        if (g < P && sub == 0) s.term0[g] = gok ? acc : 0.0f;
    } else if constexpr (TR) {
        // T2[m][k] = -2 q_m . cw_mk (ranking only: FMA allowed), built before
        // the first barrier from the query in global memory.  Every load
        // instruction reads one whole 64-byte line of each of 16 codebooks:
        // lane (m16, j) = (lane / 4, lane % 4) reads bytes 16 j .. 16 j + 15
        // of line `sp` of codebook 16 gi + m16, which hold CPS = 16 / DS
        // codewords.  With DS = 8 a codeword spans two lanes, whose partial
        // dot products meet by a lane exchange; its even lane writes it.  The
        // waves take the lines in turn, in batches of LB lines whose loads fly
        // together; batch b + 1 is issued once batch b is consumed.
        static_assert(DS == 2 || DS == 4 || DS == 8, "subvector width");
        constexpr int CPS = 16 / DS;              // codewords per line
        constexpr int LINES = KT / CPS;           // lines per codebook
        constexpr int LW = LINES / (VGPU_BLOCK / 64);  // lines per wave and codebook
        constexpr int LB = LW < 8 ? LW : 8;       // lines whose loads fly together
        static_assert(LW % LB == 0, "line batches");
        constexpr int NGI = MT / 16, NBL = LW / LB;
        const int m16 = lane >> 2, j = lane & 3;
        const int wv_ = (int)__builtin_amdgcn_readfirstlane((uint32_t)tid >> 6);
        // the query values this lane multiplies for each codebook group
        float qv[NGI][4];
#pragma unroll
        for (int gi = 0; gi < NGI; gi++) {
            const int m = gi * 16 + m16;
            if constexpr (DS == 8) load_vec<4>(a.qn + (size_t)q * D + m * 8 + 4 * (j & 1), qv[gi]);
            else if constexpr (DS == 4) load_vec<4>(a.qn + (size_t)q * D + m * 4, qv[gi]);
            else {
                load_vec<2>(a.qn + (size_t)q * D + m * 2, qv[gi]);
                qv[gi][2] = qv[gi][0];
                qv[gi][3] = qv[gi][1];
            }
        }
        // line sp = (l0 + i) * 4 + wv_ of group gi: a wave-uniform base, the
        // lane's fixed byte offset, and a constant step per line
        const uint32_t lo = (uint32_t)(m16 * KT * DS + 4 * j) * 4u;
        float4 w[LB];
        auto batch = [&](int gi, int l0) {
            const char* cbl = reinterpret_cast<const char*>(ix.codebooks + (size_t)(gi * 16) * KT * DS +
                                                            (size_t)wv_ * 16) +
                              (size_t)l0 * (VGPU_BLOCK / 64) * 64;  // wave-uniform
#pragma unroll
            for (int i = 0; i < LB; i++)
                w[i] = *reinterpret_cast<const float4*>(cbl + lo + i * (VGPU_BLOCK / 64) * 64);
        };
        batch(0, 0);
        if (tid < P) rec_load(l0id);  // in flight with the next batch; stored after its issue
#pragma unroll
        for (int gi = 0; gi < NGI; gi++) {
            // scaled by -2 (exact), so the dot products below are the table entries themselves
            float qg[4];
#pragma unroll
            for (int i = 0; i < 4; i++) qg[i] = -2.0f * qv[gi][i];
#pragma unroll 1
            for (int bl = 0; bl < NBL; bl++) {
                const int l0 = bl * LB;
                // table row of line l0 * 4 + wv_; line i of the batch is 4 i CPS rows on
                float* tl = slut + (gi * KT + (l0 * (VGPU_BLOCK / 64) + wv_) * CPS) * NC * 16 + m16;
#pragma unroll
                for (int i = 0; i < LB; i++) {
                    float* ti = tl + i * (VGPU_BLOCK / 64) * CPS * NC * 16;  // row sp * CPS
                    if constexpr (DS == 2) {
                        const float d0 = __builtin_fmaf(qg[1], w[i].y, qg[0] * w[i].x);
                        const float d1 = __builtin_fmaf(qg[3], w[i].w, qg[2] * w[i].z);
#pragma unroll
                        for (int c = 0; c < NC; c++) {
                            ti[(2 * j * NC + c) * 16] = d0;
                            ti[((2 * j + 1) * NC + c) * 16] = d1;
                        }
                    } else {
                        float dp = qg[0] * w[i].x;
                        dp = __builtin_fmaf(qg[1], w[i].y, dp);
                        dp = __builtin_fmaf(qg[2], w[i].z, dp);
                        dp = __builtin_fmaf(qg[3], w[i].w, dp);
                        int kj = j;  // codeword of the line
                        if constexpr (DS == 8) {
                            dp = add_dpp<0xB1>(dp, dp);  // + the partner half (lane j ^ 1)
                            asm volatile("" : "+v"(dp));  // every lane adds (the move folds into it)
                            kj = j >> 1;
                        }
                        if (DS != 8 || (j & 1) == 0) {
#pragma unroll
                            for (int c = 0; c < NC; c++) ti[(kj * NC + c) * 16] = dp;
                        }
                    }
                }
                if (bl + 1 < NBL) batch(gi, l0 + LB);
                else if (gi + 1 < NGI) batch(gi + 1, 0);
                if (gi == 0 && bl == 0 && tid < P) rec_store(tid);
            }
        }
        // the query itself from the slices just loaded: wave 0's lanes with
        // j < 2 (DS = 8) or j = 0 hold each dimension once
        if (tid < 64 && (DS == 8 ? j < 2 : j == 0)) {
#pragma unroll
            for (int gi = 0; gi < NGI; gi++) {
                const int m = gi * 16 + m16;
                if constexpr (DS == 8) {
#pragma unroll
                    for (int i = 0; i < 4; i++) s.qs[m * 8 + 4 * j + i] = qv[gi][i];
                } else {
#pragma unroll
                    for (int i = 0; i < DS; i++) s.qs[m * DS + i] = qv[gi][i];
                }
            }
        }
    } else {
        if (tid < P) {
            rec_load(l0id);
            rec_store(tid);
        }
        for (int jj = tid; jj < d; jj += VGPU_BLOCK) s.qs[jj] = a.qn[(size_t)q * d + jj];
    }
    for (int p = tid + VGPU_BLOCK; p < P; p += VGPU_BLOCK) {
        rec_load(a.probe[(size_t)q * P + p]);
        rec_store(p);
    }
    __syncthreads();
    if (tid < 64) {  // exclusive prefix of the list lengths (whole blocks when transposed)
        uint32_t carry = 0, entries = 0;
        for (int p0 = 0; p0 < P; p0 += 64) {
            const int p = p0 + lane;
            const uint32_t len = p < P ? s.llen[p] : 0u;
            const uint32_t own = TR ? (len + 15u) & ~15u : len;
            uint32_t x = own, y = len;
            for (int o = 1; o < 64; o <<= 1) {
                const uint32_t xs = __shfl_up(x, o, 64), ys = __shfl_up(y, o, 64);
                if (lane >= o) {
                    x += xs;
                    y += ys;
                }
            }
            if (p < P) s.pref[p] = carry + x - own;
            carry += __shfl(x, 63, 64);
            entries += __shfl(y, 63, 64);
        }
        if (lane == 0) {
            s.pref[P] = carry;
            s.misc[7] = entries;
        }
    }
    {  // ||q - c||^2: eight lanes per probed list (ranking only: any order)
        const int g = tid >> 3, sub = tid & 7;
        for (int p0 = PRE ? PG : 0; p0 < P; p0 += VGPU_BLOCK / 8) {
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
    // T2[m][k] = -2 q_m . cw_mk (ranking only: FMA allowed); the transposed
    // layout's table is built before the first barrier
    if constexpr (TR) {
    } else if constexpr (MT > 0 && KT > 0 && DS > 0 && (MT * KT) % VGPU_BLOCK == 0) {
        constexpr int NE = MT * KT / VGPU_BLOCK;           // entries per thread
        constexpr int G = DS >= 16 ? 2 : DS >= 8 ? 4 : (NE < 8 ? NE : 8);  // entries whose loads fly together
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
    __syncthreads();  // pref (wave 0) and term0 complete
    auto slot_rec = [&](int p) {
        return make_uint4(s.lbeg[p] - s.pref[p], __float_as_uint(s.term0[p]),
                          TR ? 16u * s.tbo[p] - s.pref[p] : 0u, s.pref[p] + s.llen[p]);
    };
    SlotRegs sr;  // P <= 64: lane p holds slot p's prefix sum and record
    sr.pref = lane < P ? s.pref[lane] : 0xffffffffu;
    sr.bt = lane < P ? slot_rec(lane) : make_uint4(0u, 0u, 0u, 0u);
    if (P > 64)
        for (int p = tid; p < P; p += VGPU_BLOCK) s.bt[p] = slot_rec(p);
    // The main pass's block map, when the blocks it fetches fit (block-uniform).
    bool use_map = false;
    if constexpr (kMap) {
        const uint32_t nb = s.pref[P] >> 4;               // padded blocks of the probed lists
        const uint32_t cover = ((nb + 15u) & ~15u) + 80u;  // map bytes read up to five rounds past the last
        use_map = P < 64 && cover <= (uint32_t)FS_MAP_BLOCKS;
        if (use_map) {
            FsMap& mp = aux->map;
            const int g = tid >> 3, sub = tid & 7;
            for (int p = g; p < P; p += VGPU_BLOCK / 8) {  // eight lanes per probed slot
                const uint32_t b0 = s.pref[p] >> 4, b1 = s.pref[p + 1] >> 4;  // empty lists write nothing
                for (uint32_t b = b0 + (uint32_t)sub; b < b1; b += 8u) mp.slot4[b] = (uint8_t)(4 * p);
                if (sub == 0) {
                    mp.vb16[p] = 16u * (s.tbo[p] - b0);
                    mp.t0[p] = s.term0[p];
                }
            }
            for (uint32_t b = nb + (uint32_t)tid; b < cover; b += VGPU_BLOCK) mp.slot4[b] = (uint8_t)(4 * P);
            if (tid == 0) {
                mp.vb16[P] = 0u;
                mp.t0[P] = __builtin_nanf("");
            }
        }
    }
    if (tid < 64) {  // max ||q - c||^2 for tau
        float t0max = 0.0f;
        for (int p = lane; p < P; p += 64) t0max = fmaxf(t0max, s.term0[p]);
#pragma unroll
        for (int o = 1; o < 64; o <<= 1)
            t0max = fmaxf(t0max, __uint_as_float(shfl_xor_u32(__float_as_uint(t0max), o)));
        if (lane == 0) s.misc[9] = __float_as_uint(t0max);
    }
    __syncthreads();  // llen, term0 and tbo are dead from here (they may share the key buffer)

    // ---- scan.  Wave w takes the windows rbase + 64 w (rbase = 0, FS_ROUND,
    // ...) with the next two rounds' loads in flight (a ring of three register
    // sets) and keeps its own candidates: region keys[w * BW, (w + 1) * BW), its
    // own count and filter F, and it always holds every entry the wave scanned
    // with key <= F.  F is the wave's flush threshold or the shared bound
    // misc[8], whichever is lower.  A flush's T is the keep-th smallest key the
    // wave has seen (keep >= kout), an upper bound on the query's final A_k, so
    // no entry above T + 2 tau belongs to R; each flush publishes that bound.
    // No barrier until the end of the scan.
    const uint32_t total = s.pref[P];
    const int keep = a.kk;
    const uint32_t BW = (uint32_t)buf / (VGPU_BLOCK / 64);  // region capacity
    const uint32_t capw = BW - 64u;
    const uint32_t wave = __builtin_amdgcn_readfirstlane((uint32_t)tid >> 6);
    uint64_t* reg = s.keys + wave * BW;
    const float tau = fast_tau(d, M, ds, a.qnorm[q], ix.cmax, ix.rmax, __uint_as_float(s.misc[9]));
    uint32_t cnt = 0, thr = 0xffffffffu, F = 0xffffffffu, Fused = 0xffffffffu, evicted = 0, flushes = 0;
    bool lost = false;
    int cur = 0;
    RoundRegs<MT> ga, gb, gc, gd;
    // transposed blocks as lane records (unused by the row layout)
    const __amdgpu_buffer_rsrc_t rsc = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint8_t*>(ix.tcodes), (short)(TR ? MT : 0), (int)(TR ? 16u * ix.tblk_count : 0u), 0x00020000);
    const __amdgpu_buffer_rsrc_t rsb = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<float*>(ix.tbias), (short)4, (int)(TR ? 16u * ix.tblk_count : 0u), 0x00020000);
    const bool packed = TR && P <= 64 && total < (1u << FS_LBL_BITS);  // wave-uniform
    auto fetch = [&](uint32_t rb, RoundRegs<MT>& g) {
        if constexpr (TR) fs8t_fetch<MT>(rsc, rsb, s, sr, rb, P, cur, g, packed);
        else fs8_fetch<MT>(ix, s, sr, rb, total, P, cur, g);
    };
    MapPipe mpp{0u, 0u, 0u, 0.0f};
    if (kMap && use_map) {  // the record of round 0 and the map byte of round 1
        fs8m_record(aux->map, 0u, fs8m_byte(aux->map, 0u), mpp);
        mpp.s4n = fs8m_byte(aux->map, FS_ROUND);
    }
    auto mfetch = [&](uint32_t rb, RoundRegs<MT>& g) {
        if constexpr (kMap) fs8m_fetch<MT>(rsc, rsb, aux->map, rb, mpp, g);
    };
    // Whole groups of four rounds in the loop, which has no other exit (an
    // exit inside would make the loads of its first round look outstanding
    // at the loop head and drain the ring there), then the last 0 .. 3.
    const uint32_t nr = (total + FS_ROUND - 1) / FS_ROUND;  // rounds
    auto main_pass = [&](auto&& fetchf) {
    if (total > 0) {
        fetchf(0, ga);
        fetchf(FS_ROUND, gb);
        fetchf(2 * FS_ROUND, gc);
    }
#define FS8_STEP(CONSUME, NEXT, R)                                                           \
    {                                                                                        \
        const uint32_t rbase = (R) * FS_ROUND;                                               \
        fetchf(rbase + 3 * FS_ROUND, NEXT);                                                  \
        const uint32_t shared = __atomic_load_n(&s.misc[8], __ATOMIC_RELAXED);               \
        Fused = F;                                                                           \
        fs8w_consume<MT, KT, NC>(ix, s, slut, CONSUME, filter_float(F), reg, cnt);           \
        if (cnt > capw) {                                                                    \
            const uint32_t before = cnt;                                                     \
            thr = fs8w_flush(reg, cnt, (uint32_t)keep - 1u, capw, &lost);                    \
            evicted += before - cnt;                                                         \
            flushes++;                                                                       \
            uint32_t ub = fkey(fkey_to_float(thr) + 2.0f * tau);                             \
            ub = ub < 0xfffffffeu ? ub + 1u : 0xffffffffu;                                   \
            if (thr < 0xff800000u && lane == 0) atomicMin(&s.misc[8], ub);                   \
        }                                                                                    \
        {   /* the next round's filter (the bound read before this round's lookups) */        \
            const uint32_t sh = __builtin_amdgcn_readfirstlane(shared);                      \
            F = thr < sh ? thr : sh;                                                         \
        }                                                                                    \
    }
    uint32_t r = 0;
    for (; r + 4 <= nr; r += 4) {
        FS8_STEP(ga, gd, r)
        FS8_STEP(gb, ga, r + 1)
        FS8_STEP(gc, gb, r + 2)
        FS8_STEP(gd, gc, r + 3)
    }
    if (r < nr) {
        FS8_STEP(ga, gd, r)
        if (r + 1 < nr) {
            FS8_STEP(gb, ga, r + 1)
            if (r + 2 < nr) FS8_STEP(gc, gb, r + 2)
        }
    }
#undef FS8_STEP
    };
    if (kMap && use_map) main_pass(mfetch);
    else main_pass(fetch);
    {
        const uint32_t G = Fused < thr ? Fused : thr;  // the wave's region holds its entries <= G
        if (lane == 0) {
            s.misc[16 + wave] = cnt;
            s.misc[20 + wave] = G;
            atomicAdd(&s.misc[5], evicted);
            atomicAdd(&s.misc[6], flushes);
            if (lost) s.misc[2] = 1u;
        }
    }
    __syncthreads();

    // ---- proof that the merged buffer holds R, then rescoring.
    uint32_t cnts[VGPU_BLOCK / 64];
    uint32_t thr_all = 0xffffffffu;  // every wave holds its entries <= thr_all
#pragma unroll
    for (int w = 0; w < VGPU_BLOCK / 64; w++) {
        cnts[w] = s.misc[16 + w];
        const uint32_t g = s.misc[20 + w];
        thr_all = g < thr_all ? g : thr_all;
    }
    const uint32_t Gw = s.misc[20 + wave];
    // Dense index i of the waves' keys: wave w's keys are roff[w] .. roff[w + 1],
    // read in place until a second pass needs them merged.
    uint32_t roff[VGPU_BLOCK / 64 + 1];
    roff[0] = 0;
#pragma unroll
    for (int w = 0; w < VGPU_BLOCK / 64; w++) roff[w + 1] = roff[w] + cnts[w];
    uint32_t n = roff[VGPU_BLOCK / 64];
    bool merged = false;
    auto key_at = [&](uint32_t i) -> uint64_t { return s.keys[merged ? i : region_slot(i, roff, BW)]; };
    const uint32_t cap = (uint32_t)buf - FS_ROUND;  // second-pass capacity
    const int kout = a.kout;
    bool fail = s.misc[2] != 0u;
    bool retried = false;
    uint32_t bk = 0xffffffffu;
    if (!fail && n > (uint32_t)kout) {
        // an upper bound on A_k: R grows by at most the rest of A_k's bin
        const uint32_t Ak = fs8_select_upper(s, key_at, n, (uint32_t)(kout - 1), 0xffffffffu);
        const float bound = fkey_to_float(Ak) + 2.0f * tau;
        bk = fkey(bound);
        bk = bk < 0xfffffffeu ? bk + 1u : 0xffffffffu;  // one ulp to spare
        if (thr_all != 0xffffffffu && bk > thr_all) {
            // Second pass: wave w's entries <= G_w are held; each wave adds
            // its entries in (G_w, bk] with no flush, so afterwards the buffer
            // holds all of R.  More than the buffer holds fails the query
            // (EXACT rerun).
            retried = true;
            n = fs8w_merge(s, cnts, BW);
            merged = true;
            if (tid == 0) {
                s.misc[0] = n;
                s.misc[3] = s.misc[4] = 0u;
            }
            __syncthreads();
            cur = 0;
            fetch(0, ga);
            for (uint32_t rb = 0; rb < total; rb += 2 * FS_ROUND) {
                fetch(rb + FS_ROUND, gb);
                fs8_consume_retry<MT, KT, NC>(ix, s, slut, ga, bk, Gw, cap, 0);
                __syncthreads();
                if (s.misc[3]) break;
                if (rb + FS_ROUND >= total) break;
                fetch(rb + 2 * FS_ROUND, ga);
                fs8_consume_retry<MT, KT, NC>(ix, s, slut, gb, bk, Gw, cap, 1);
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
        st[0] = s.misc[7];  // list entries, without block padding
        st[1] = s.misc[6];
        st[2] = s.misc[5] + n;  // appended = evicted + still held
        st[3] = (fail ? (1u | (s.misc[2] ? 2u : 0u)) : 0u) | (retried ? 4u : 0u);
        if (fail) a.flag_list[atomicAdd(a.flag_count, 1u)] = (uint32_t)q;
    }
    if (fail) return;
    // The table is no longer needed: the residuals r = q - c of the probed
    // lists go to its region now (their loads overlap the compaction) when
    // the two-thread rescoring below may use them.  Thread t stages
    // dimensions 4 (t % (D / 4)) .. + 3 of slots t / (D / 4), + SPT, ...: the
    // slot ids are read first and every centroid load is in flight at once
    // (a store to the table region could otherwise hold back the next id read).
    if constexpr ((MT == 8 || MT == 16 || MT == 32) && KT > 0 && DS > 0) {
        if ((size_t)P * D <= (size_t)LUTF) {
            constexpr int SPT = VGPU_BLOCK / (D / 4);         // slots per pass
            constexpr int SMAX = (LUTF / D + SPT - 1) / SPT;  // passes for P D <= LUTF
            static_assert(D % 4 == 0, "staging split");
            // threads past the pass's SPT whole slots stage nothing
            const int j = 4 * (tid % (D / 4)), pp0 = tid < SPT * (D / 4) ? tid / (D / 4) : P;
            uint32_t lr[SMAX];
#pragma unroll
            for (int it = 0; it < SMAX; it++) lr[it] = pp0 + it * SPT < P ? s.lid[pp0 + it * SPT] : 0u;
            const float4 qv = *reinterpret_cast<const float4*>(a.qn + (size_t)q * D + j);
            float4 c[SMAX];
#pragma unroll
            for (int it = 0; it < SMAX; it++)
                if (pp0 + it * SPT < P) c[it] = *reinterpret_cast<const float4*>(ix.centroids + (size_t)lr[it] * D + j);
#pragma unroll
            for (int it = 0; it < SMAX; it++) {
                const int pp = pp0 + it * SPT;
                if (pp < P) {
                    float* o = s.lut + pp * D + j;
                    o[0] = __fsub_rn(qv.x, c[it].x);
                    o[1] = __fsub_rn(qv.y, c[it].y);
                    o[2] = __fsub_rn(qv.z, c[it].z);
                    o[3] = __fsub_rn(qv.w, c[it].w);
                }
            }
        }
    }
    // Regions in place and residuals staged: each wave keeps the keys of its
    // own region that belong to R, relabelled, at the front of its region
    // (no block barrier; an odd count is followed by a key above every other,
    // for the pairwise reads of the ordering).  R is then rescored where it
    // lies, two threads per entry with the exact distance below, and ordered
    // across the regions without merging them.
    if constexpr ((MT == 8 || MT == 16 || MT == 32) && KT > 0 && DS > 0) {
        if ((size_t)P * D <= (size_t)LUTF && !merged) {
            const uint32_t cntw = cnts[wave];
            uint32_t kept = 0;
            for (uint32_t i0 = 0; i0 < cntw; i0 += 64) {  // chunk read before any slot of it is rewritten
                const uint32_t idx = i0 + (uint32_t)lane;
                uint64_t v = idx < cntw ? reg[idx] : ~0ull;
                const bool take = idx < cntw && (uint32_t)(v >> 32) <= bk;
                const uint64_t mask = __ballot(take);
                if (take) {
                    v = fs8_relabel(s, v, P, packed);
                    reg[kept + __builtin_amdgcn_mbcnt_hi((uint32_t)(mask >> 32),
                                                         __builtin_amdgcn_mbcnt_lo((uint32_t)mask, 0u))] = v;
                }
                kept += (uint32_t)__popcll(mask);
            }
            if (lane == 0) {
                s.misc[16 + wave] = kept;
                if (kept & 1u) reg[kept] = ~0ull;  // kept < capw < BW
            }
            __syncthreads();  // residuals staged, R final in every region
            uint32_t ro[VGPU_BLOCK / 64 + 1];
            ro[0] = 0;
#pragma unroll
            for (int w = 0; w < VGPU_BLOCK / 64; w++) ro[w + 1] = ro[w] + s.misc[16 + w];
            n = ro[VGPU_BLOCK / 64];
            for (uint32_t c0 = 0; c0 < n; c0 += VGPU_BLOCK / 2) {
                const uint32_t i = c0 + ((uint32_t)tid >> 1), half = (uint32_t)tid & 1u;
                const bool act = i < n;
                const uint32_t at = act ? region_slot(i, ro, BW) : 0u;
                const uint64_t v = act ? s.keys[at] : 0ull;
                const uint32_t vid = act && half == 0 ? ix.list_ids[(uint32_t)v] : 0u;
                CodeRow<MT> row;  // both lanes of the pair hold the whole row (entry 0 when inactive)
                load_row<MT>(row, ix.codes + (size_t)(uint32_t)v * MT);
                const float total_e =
                    fs8_pair_distance<MT, KT, DS, MT <= 16 ? 4 : 2>(ix, s.lut, (uint32_t)(v >> 32), row, half);
                if (act && half == 0) s.keys[at] = cand_key(total_e, vid);  // its own slot: no other reads it
            }
            __syncthreads();
            if (n <= (uint32_t)VGPU_BLOCK) {
                // Each thread takes one key and writes it at its rank, the number
                // of smaller keys over the regions (distinct keys: one per
                // vector); its doc id load flies during the count.
                if ((uint32_t)tid < n) {
                    const uint64_t ki = s.keys[region_slot((uint32_t)tid, ro, BW)];
                    const uint32_t vi = (uint32_t)ki;
                    const uint32_t doc = a.out_ids && a.doc_ids ? a.doc_ids[vi] : vi;
                    uint32_t r = 0;
#pragma unroll
                    for (int w = 0; w < VGPU_BLOCK / 64; w++) {
                        const uint64_t* rk = s.keys + (uint32_t)w * BW;
                        const uint32_t cw2 = ro[w + 1] - ro[w];
#pragma unroll 4
                        for (uint32_t jj = 0; jj < cw2; jj += 2) {
                            const ulonglong2 kj = *reinterpret_cast<const ulonglong2*>(rk + jj);
                            r += (kj.x < ki ? 1u : 0u) + (kj.y < ki ? 1u : 0u);
                        }
                    }
                    if (r < (uint32_t)kout) {
                        const size_t o = (size_t)q * kout + r;
                        if (a.out_ids) {
                            a.out_ids[o] = (int64_t)doc;
                            a.out_dists[o] = key_dist(ki);
                        } else {
                            a.out_vidx[o] = vi;
                            a.out_dist[o] = key_dist(ki);
                        }
                    }
                }
                for (int j = (int)n + tid; j < kout; j += VGPU_BLOCK) scan_emit(a, q, j, ~0ull, false);  // padding
                return;
            }
            uint32_t kc[VGPU_BLOCK / 64];
#pragma unroll
            for (int w = 0; w < VGPU_BLOCK / 64; w++) kc[w] = ro[w + 1] - ro[w];
            n = fs8w_merge(s, kc, BW);
            goto rescored;
        }
    }
    n = fs8_compact(s, key_at, n, bk, true, P, packed);  // R, keys relabelled (probe slot, position)

    // Two threads per entry (codebooks 0 .. M/2 - 1 and M/2 .. M - 1) when the
    // probed lists' residuals r = q - c fit the idle table region (built
    // above): each thread loads its half code row (and the first thread the
    // entry's insertion index), then all its codewords at once (at most 64
    // floats); r comes from LDS (the same single subtraction
    // exact_sub_distance makes).  The first
    // thread adds its sub-distances in codebook order from 0.0 and continues
    // with its partner's, handed over by a lane shuffle (pq_simd.rs:349-355).
    if constexpr (MT == 8 || MT == 16 || MT == 32) {
        if constexpr (KT > 0 && DS > 0) {
            if ((size_t)P * D <= (size_t)LUTF && n <= (uint32_t)(VGPU_BLOCK / 2)) {
                const uint32_t i = (uint32_t)tid >> 1, half = (uint32_t)tid & 1u;
                const bool act = i < n;
                const uint64_t v = act ? s.keys[i] : 0ull;
                const uint32_t vid = act && half == 0 ? ix.list_ids[(uint32_t)v] : 0u;
                CodeRow<MT> row;  // both lanes of the pair hold the whole row (entry 0 when inactive)
                load_row<MT>(row, ix.codes + (size_t)(uint32_t)v * MT);
                // fewer codewords in flight for wide rows (registers)
                const float total_e = fs8_pair_distance<MT, KT, DS, MT <= 16 ? 4 : 2>(
                    ix, s.lut, (uint32_t)(v >> 32), row, half);
                __syncthreads();  // every key of R read above before any is rewritten
                if (act && half == 0) s.keys[i] = cand_key(total_e, vid);
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
            s.lut[t] = exact_sub_distance<DS>(a.qn + (size_t)q * d + m * ds, c, cw, ds);
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
    if (n <= (uint32_t)VGPU_BLOCK) {
        // Each thread takes one key and writes it at its position in the
        // ascending order, the number of smaller keys (the keys are distinct:
        // one per vector); its doc id load flies during the count.
        if (tid == 0 && (n & 1u)) s.keys[n] = ~0ull;  // even count for the pairwise reads; above every key
        __syncthreads();
        if ((uint32_t)tid < n) {
            const uint64_t ki = s.keys[tid];
            const uint32_t vi = (uint32_t)ki;
            const uint32_t doc = a.out_ids && a.doc_ids ? a.doc_ids[vi] : vi;
            uint32_t r = 0;
#pragma unroll 8
            for (uint32_t jj = 0; jj < n; jj += 2) {
                const ulonglong2 kj = *reinterpret_cast<const ulonglong2*>(s.keys + jj);
                r += (kj.x < ki ? 1u : 0u) + (kj.y < ki ? 1u : 0u);
            }
            if (r < (uint32_t)kout) {
                const size_t o = (size_t)q * kout + r;
                if (a.out_ids) {
                    a.out_ids[o] = (int64_t)doc;
                    a.out_dists[o] = key_dist(ki);
                } else {
                    a.out_vidx[o] = vi;
                    a.out_dist[o] = key_dist(ki);
                }
            }
        }
        for (int j = (int)n + tid; j < kout; j += VGPU_BLOCK) scan_emit(a, q, j, ~0ull, false);  // padding
        return;
    }
    const int n2 = next_pow2((int)n);
    for (int t = (int)n + tid; t < n2; t += VGPU_BLOCK) s.keys[t] = ~0ull;
    block_bitonic_sort_keys(s.keys, n2);
    for (int j = tid; j < kout; j += VGPU_BLOCK) scan_emit(a, q, j, s.keys[j], (uint32_t)j < n);
}

// ---- per-query tables for a chunk of queries -----------------------------
// T2[q][(16 gi + r) codebook, c codeword] = -2 q_m . cw_mc (m = 16 gi + r)
// at float ((gi * 256 + c) * 16 + r) of query q's M * 256 floats: the layout
// of the FAST scan's LDS table (transposed blocks, one copy).  Ranking only,
// like the table the scan builds itself: the dot products are fp32 MFMA
// (v_mfma_f32_16x16x4_f32, products of fp32 operands summed in fp32), within
// 2 ds u sum_j |q_j cw_j| of the real ones even if the sums truncate, which
// the error bound fast_tau covers.  One workgroup per (16 queries, 16
// codewords of a 16-codebook group).  The queries' slices of the group and
// the tile's codewords (16 ds floats per row, contiguous in both arrays) are
// staged in LDS with coalesced 16-byte loads, one dimension step padded to 4
// per codebook; wave w then computes codebooks 4 w .. 4 w + 3 (A = the query
// values scaled by -2, exact; B = the codewords).  The 16 x 16 x 16 results
// are staged in LDS and stored with each instruction covering 4 KB of
// consecutive bytes (one kilobyte per query).  Loading the operands straight
// from global memory, four bytes per lane, took 2.4x as long.
template <int DS>
__global__ __launch_bounds__(256) void t2_table_kernel(const float* __restrict__ qn, int nq, int M,
                                                       const float* __restrict__ cb, float* __restrict__ t2) {
    typedef float floatx4 __attribute__((ext_vector_type(4)));
    constexpr int KS = (DS + 3) / 4;  // MFMA steps of 4 dimensions
    constexpr int DP = KS * 4;        // padded dimensions per codebook
    constexpr int RS = 16 * DP + 4;   // LDS row stride (+4: the 16 rows of an operand read in distinct banks)
    constexpr int RF = 16 * DS / 4;   // 16-byte pieces per operand row
    static_assert(DS % 2 == 0, "even subvector widths");
    __shared__ __align__(16) float stage[16 * 256];  // [query][codeword][codebook r]
    __shared__ __align__(16) float sa[16 * RS];      // [query][codebook * DP + k]
    __shared__ __align__(16) float sb[16 * RS];      // [codeword][codebook * DP + k]
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int tiles = (M / 16) * 16;
    const int qb = blockIdx.x / tiles, gt = blockIdx.x % tiles, gi = gt >> 4, ct = gt & 15;
    const int q0 = qb * 16;
    const int i = lane & 15, kq = lane >> 4;  // A row / B column i, dimension 4 step + kq
    const int rows = min(16, nq - q0);
    const int d = M * DS;
    if (DP != DS)
        for (int f = tid; f < 16 * RS; f += VGPU_BLOCK) sa[f] = sb[f] = 0.0f;  // the padded dimensions
    __syncthreads();
    for (int f = tid; f < 16 * RF; f += VGPU_BLOCK) {
        const int r = f / RF, c4 = f % RF, m = 4 * c4 / DS, k = 4 * c4 % DS;
        float4 x = make_float4(0.f, 0.f, 0.f, 0.f);
        if (r < rows) x = reinterpret_cast<const float4*>(qn + (size_t)(q0 + r) * d + (size_t)gi * 16 * DS)[c4];
        const float4 y = reinterpret_cast<const float4*>(cb + ((size_t)(16 * gi + r) * 256 + 16 * ct) * DS)[c4];
        const int cw = 4 * c4 / DS;  // B: row r is codebook 16 gi + r, piece c4 is codeword cw, dims k..
        if constexpr (DS == 2) {     // a piece spans two codebooks (A) or two codewords (B)
            sa[r * RS + m * DP] = x.x;
            sa[r * RS + m * DP + 1] = x.y;
            sa[r * RS + (m + 1) * DP] = x.z;
            sa[r * RS + (m + 1) * DP + 1] = x.w;
            sb[cw * RS + r * DP] = y.x;
            sb[cw * RS + r * DP + 1] = y.y;
            sb[(cw + 1) * RS + r * DP] = y.z;
            sb[(cw + 1) * RS + r * DP + 1] = y.w;
        } else if constexpr (DS % 4 == 0) {
            *reinterpret_cast<float4*>(sa + r * RS + m * DP + k) = x;
            *reinterpret_cast<float4*>(sb + cw * RS + r * DP + (4 * c4 % DS)) = y;
        } else {  // DS = 6: a piece may span two codebooks (A) or two codewords (B)
            const float xv[4] = {x.x, x.y, x.z, x.w}, yv[4] = {y.x, y.y, y.z, y.w};
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const int jj = 4 * c4 + e;  // float of the row: codebook / codeword jj / DS, dimension jj % DS
                sa[r * RS + (jj / DS) * DP + jj % DS] = xv[e];
                sb[(jj / DS) * RS + r * DP + jj % DS] = yv[e];
            }
        }
    }
    __syncthreads();
    floatx4 acc[4];
#pragma unroll
    for (int r = 0; r < 4; r++) {
        const int m = 4 * wave + r;
        acc[r] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int st = 0; st < KS; st++)
            acc[r] = __builtin_amdgcn_mfma_f32_16x16x4f32(-2.0f * sa[i * RS + m * DP + 4 * st + kq],
                                                          sb[i * RS + m * DP + 4 * st + kq], acc[r], 0, 0, 0);
    }
    // acc[r][e]: query 4 kq + e, codeword 16 ct + i, codebook 16 gi + 4 wave + r
#pragma unroll
    for (int e = 0; e < 4; e++)
        *reinterpret_cast<float4*>(stage + ((4 * kq + e) * 16 + i) * 16 + 4 * wave) =
            make_float4(acc[0][e], acc[1][e], acc[2][e], acc[3][e]);
    __syncthreads();
    const size_t per_q = (size_t)M * 256;
    const float4* src = reinterpret_cast<const float4*>(stage);
#pragma unroll
    for (int v = 0; v < 4; v++) {  // piece f of the tile: query f / 64, its 16 bytes f % 64
        const int f = v * VGPU_BLOCK + tid, qq = f >> 6;
        if (qq < rows)
            reinterpret_cast<float4*>(t2 + (size_t)(q0 + qq) * per_q + (size_t)(gi * 256 + 16 * ct) * 16)[f & 63] =
                src[f];
    }
}

bool scan8_fast_uses_tables(const DevIndex& ix) {
    return ix.tcodes && ix.K == 256 && ix.M == 16 && (ix.ds == 2 || ix.ds == 4 || ix.ds == 6 || ix.ds == 8);
}

void launch_t2_tables(const DevIndex& ix, const float* qn, int nq, float* t2, hipStream_t s, hipEvent_t t0,
                      hipEvent_t t1) {
    if (nq <= 0) return;
    const dim3 grid((unsigned)((size_t)((nq + 15) / 16) * (size_t)(ix.M / 16) * 16)), block(VGPU_BLOCK);
    auto go = [&](auto k) {
        if (t0) hipExtLaunchKernelGGL(k, grid, block, 0, s, t0, t1, 0u, qn, nq, ix.M, ix.codebooks, t2);
        else hipLaunchKernelGGL(k, grid, block, 0, s, qn, nq, ix.M, ix.codebooks, t2);
    };
    switch (ix.ds) {
        case 2: go(t2_table_kernel<2>); return;
        case 4: go(t2_table_kernel<4>); return;
        case 6: go(t2_table_kernel<6>); return;
        default: go(t2_table_kernel<8>); return;
    }
}

// Width 6 only with 16 codebooks, whose scan takes its table from the pre-pass
// (the scan's own transposed table build reads 64-byte lines of 2, 4 or 8).
bool scan8_fast_blocks_supported(int M, int K, int ds) {
    return K == 256 && (((M == 16 || M == 32 || M == 48) && (ds == 2 || ds == 4 || ds == 8)) || (M == 16 && ds == 6));
}

// Table copies of the transposed kernels (0: row layout).  One copy: with
// 16 codebooks two copies would let a half wave read 32 distinct banks, but
// the doubled table costs more in occupancy than the conflicts it removes.
static int table_copies(const DevIndex& ix) {
    return ix.tcodes && scan8_fast_blocks_supported(ix.M, ix.K, ix.ds) ? 1 : 0;
}

// Static table bytes of the specialisations (compile-time M, K = 256).
static size_t static_lut_bytes(const DevIndex& ix) {
    if (ix.K != 256) return 0;
    const int nc = table_copies(ix);
    switch (ix.M) {
        case 4: case 8: case 16: case 32: case 48: case 64:
            return (size_t)ix.M * 256 * 4 * (nc ? nc : 1);
        default: return 0;
    }
}

size_t scan8_fast_lds_bytes(const DevIndex& ix, const ScanArgs& a) {
    size_t off[12];
    const size_t st = static_lut_bytes(ix);
    // the block map's static LDS (in place of the dynamic radix scratch)
    const bool map = st != 0 && fs8_has_map(ix.M, table_copies(ix));
    return st + (map ? (sizeof(FsAux) + 15) & ~(size_t)15 : 0) + fs8_layout(ix.d, ix.M, ix.K, a.P, fs8_buf(a.kk), st != 0, off, map);
}

template <int MT, int KT, int DS, int NC, int PRE = 0>
static void launch_fast(const DevIndex& ix, const ScanArgs& a, hipStream_t s, hipEvent_t t0,
                        hipEvent_t t1) {
    const int buf = fs8_buf(a.kk);
    size_t off[12];
    const size_t dyn = fs8_layout(ix.d, ix.M, ix.K, a.P, buf, MT > 0 && KT >= 64, off, fs8_has_map(MT, NC));
    auto k = scan8_fast_kernel<MT, KT, DS, NC, PRE>;
    ensure_dyn_lds((const void*)k, dyn);
    if (t0)
        hipExtLaunchKernelGGL(k, dim3(a.nq), dim3(VGPU_BLOCK), (uint32_t)dyn, s, t0, t1, 0u, ix, a, buf);
    else
        hipLaunchKernelGGL(k, dim3(a.nq), dim3(VGPU_BLOCK), dyn, s, ix, a, buf);
}

// Compile-time subvector width; the shapes with transposed blocks use them.
template <int MT, int DS>
static void launch_fast_ds(const DevIndex& ix, const ScanArgs& a, hipStream_t s, hipEvent_t t0,
                           hipEvent_t t1) {
    if constexpr (MT == 16 || MT == 32 || MT == 48) {
        if constexpr (MT == 16)
            if (table_copies(ix) == 1 && a.t2) return launch_fast<MT, 256, DS, 1, 1>(ix, a, s, t0, t1);
        if (table_copies(ix) == 1) return launch_fast<MT, 256, DS, 1>(ix, a, s, t0, t1);
        return launch_fast<MT, 256, 0, 0>(ix, a, s, t0, t1);  // blocks missing: row layout
    } else {
        launch_fast<MT, 256, DS, 0>(ix, a, s, t0, t1);
    }
}

// Subvector widths 3, 6, 12 and 16 (d 96 or 48 with 8, 16 or 32 codebooks,
// d 128 or 64 with 8 or 4, ...): the row layout with the width fixed at
// compile time, which scanned d 96 about twice as fast as the run-time width.  Up to 32 codebooks and d 192;
// 16 codebooks of 12 (d 192) spilled and take the run-time width, as do the
// rest.  With 16 codebooks of 6 (d 96) the transposed blocks and the
// pre-pass tables serve the scan instead.
template <int MT, int DS>
static void launch_fast_row(const DevIndex& ix, const ScanArgs& a, hipStream_t s, hipEvent_t t0,
                            hipEvent_t t1) {
    if constexpr (MT == 16 && DS == 6)  // d 96: transposed blocks with the pre-pass tables
        if (table_copies(ix) == 1 && a.t2) return launch_fast<MT, 256, DS, 1, 1>(ix, a, s, t0, t1);
    if constexpr (MT <= 32 && MT * DS <= 192 && !(MT == 16 && DS == 12)) launch_fast<MT, 256, DS, 0>(ix, a, s, t0, t1);
    else launch_fast<MT, 256, 0, 0>(ix, a, s, t0, t1);
}

template <int MT>
static void launch_fast_m(const DevIndex& ix, const ScanArgs& a, hipStream_t s, hipEvent_t t0,
                          hipEvent_t t1) {
    switch (ix.ds) {  // the subvector widths of the benchmark shapes
        case 2: launch_fast_ds<MT, 2>(ix, a, s, t0, t1); return;
        case 4: launch_fast_ds<MT, 4>(ix, a, s, t0, t1); return;
        case 8: launch_fast_ds<MT, 8>(ix, a, s, t0, t1); return;
        case 3: launch_fast_row<MT, 3>(ix, a, s, t0, t1); return;
        case 6: launch_fast_row<MT, 6>(ix, a, s, t0, t1); return;
        case 12: launch_fast_row<MT, 12>(ix, a, s, t0, t1); return;
        case 16: launch_fast_row<MT, 16>(ix, a, s, t0, t1); return;
        default: launch_fast<MT, 256, 0, 0>(ix, a, s, t0, t1); return;
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
    launch_fast<0, 0, 0, 0>(ix, a, s, t0, t1);
}


}  // namespace vgpu
