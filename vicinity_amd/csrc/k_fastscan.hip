// 4-bit FastScan scan (codebook_size == 16), one workgroup per query, one
// wave per probed list.
//
// Reference: search.rs:1261-1287 (lists of >= 16 entries take FastScan, the
// rest the exact float path :1355-1375); quantize_lut_flat
// src/pq_simd.rs:576-611 (global min/max, scale = range/255, inv = 255/range,
// round half away from zero, clamp); fastscan_block_portable :629-654 (u16
// accumulation); fastscan_batch_quantized :721-769 (acc * scale + offset * M);
// PackedCodes4bit layout :426-486 (32-entry blocks, per codebook 16 bytes,
// byte[lane] = code[lane] | code[lane + 16] << 4).
//
// The quantised table of one codebook is 16 bytes = 4 dwords; a packed dword
// holds the nibbles of 8 entries, looked up 4 at a time with v_perm_b32
// (byte select from a 64-bit pair) and accumulated as packed u16 pairs, which
// cannot carry across halves because M <= 257 keeps every sum <= 65535.
#include "vgpu_device.h"
#include "vgpu_launch.h"

namespace vgpu {

__device__ __forceinline__ void wave_sync() {
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
    __builtin_amdgcn_wave_barrier();
}

// Round half away from zero, then Rust's saturating f32 -> u8 cast.
__device__ __forceinline__ uint32_t round_to_u8(float v) {
    float r = roundf(v);
    if (!(r >= 0.0f)) return 0u;
    if (r > 255.0f) return 255u;
    return (uint32_t)r;
}

// Accumulate one codebook of one packed dword (8 entries) into four packed
// u16 pairs: a0 = entries (4w, 4w+2), a1 = (4w+1, 4w+3), a2/a3 the same + 16.
// Each byte's index selects from the table's low (t0, t1) or high (t2, t3)
// 8 bytes by its bit 3.  That byte mask comes from v_perm_b32's
// sign-replicating selectors (8..11 give 0xff when bit 15, 31, 47 or 63 of
// the source pair is set), straight from x: bit 3 of the low nibbles sits
// at bits 3, 11, 19, 27 (brought to those bits by x << 4 and x << 12), bit 3
// of the high nibbles at bits 7, 15, 23, 31 (x and x << 8).  Odd bytes move
// to u16 slots by a byte select against zero (selector 0x0c gives 0x00).
__device__ __forceinline__ void fs_accumulate(uint32_t x, uint32_t t0, uint32_t t1, uint32_t t2,
                                              uint32_t t3, uint32_t& a0, uint32_t& a1,
                                              uint32_t& a2, uint32_t& a3) {
    const uint32_t il = x & 0x07070707u, ih = (x >> 4) & 0x07070707u;
    const uint32_t ml = __builtin_amdgcn_perm(x << 12, x << 4, 0x090b080au);
    const uint32_t mh = __builtin_amdgcn_perm(x << 8, x, 0x090b080au);
    const uint32_t rl = (__builtin_amdgcn_perm(t3, t2, il) & ml) | (__builtin_amdgcn_perm(t1, t0, il) & ~ml);
    const uint32_t rh = (__builtin_amdgcn_perm(t3, t2, ih) & mh) | (__builtin_amdgcn_perm(t1, t0, ih) & ~mh);
    a0 += rl & 0x00ff00ffu;
    a1 += __builtin_amdgcn_perm(0u, rl, 0x0c030c01u);
    a2 += rh & 0x00ff00ffu;
    a3 += __builtin_amdgcn_perm(0u, rh, 0x0c030c01u);
}

// u16 accumulator of entry c (0..7) of a lane: c -> vector 4w + c (c < 4) or
// 16 + 4w + (c - 4).
__device__ __forceinline__ uint32_t fs_acc(int c, uint32_t a0, uint32_t a1, uint32_t a2,
                                           uint32_t a3) {
    switch (c) {
        case 0: return a0 & 0xffffu;
        case 1: return a1 & 0xffffu;
        case 2: return a0 >> 16;
        case 3: return a1 >> 16;
        case 4: return a2 & 0xffffu;
        case 5: return a3 & 0xffffu;
        case 6: return a2 >> 16;
        default: return a3 >> 16;
    }
}

// Wave-level quantisation (quantize_lut_flat, pq_simd.rs:576-611) of the
// float table whose entry e is value_of(e), e < M * 16, into qlut (bytes):
// min and max over the entries, then each entry again for its byte.
template <typename V>
__device__ inline void fs_quantize_entries(V value_of, uint8_t* qlut, int M, float& scale, float& base_offset) {
    const int lane = threadIdx.x & 63;
    float mn = __int_as_float(0x7f800000), mx = __int_as_float(0xff800000);
    for (int e = lane; e < M * 16; e += 64) {
        const float v = value_of(e);
        if (v < mn) mn = v;
        if (v > mx) mx = v;
    }
    for (int off = 32; off > 0; off >>= 1) {
        float omn = __shfl_xor(mn, off, 64), omx = __shfl_xor(mx, off, 64);
        if (omn < mn) mn = omn;
        if (omx > mx) mx = omx;
    }
    float range = mx - mn;
    float sc, inv;
    if (range < 1.1920929e-07f) {
        sc = 1.0f;
        inv = 0.0f;
    } else {
        sc = range / 255.0f;
        inv = 255.0f / range;
    }
    for (int e = lane; e < M * 16; e += 64) qlut[e] = (uint8_t)round_to_u8((value_of(e) - mn) * inv);
    scale = sc;
    base_offset = mn * (float)M;
}

// A float table held in LDS.
__device__ inline void fs_quantize(const float* lutf, uint8_t* qlut, int M, float& scale, float& base_offset) {
    fs_quantize_entries([&](int e) { return lutf[e]; }, qlut, M, scale, base_offset);
}

// Codebooks of at most this many bytes are staged in LDS once per query for
// the table builds; larger ones are read from global memory.
#define FS_CB_LDS 16384
#define FS_CW 16  // codebooks whose code words a lane loads together
__host__ __device__ inline bool fs_cb_in_lds(int M, int ds) { return (size_t)M * 16 * ds * 4 <= FS_CB_LDS; }

// Entry e = m * 16 + c of the float table of residual rw:
// sum_j (r_mj - cw_mcj)^2 in j order (pq.rs:232-251).
__device__ __forceinline__ float fs_lut_value(const float* rw, const float* cb, int ds, int e) {
    if (ds == 2) {  // straight-line: one 8-byte read of each operand, the same sum
        const float2 c2 = *reinterpret_cast<const float2*>(cb + (size_t)e * 2);
        const float2 r2 = *reinterpret_cast<const float2*>(rw + (e >> 4) * 2);
        const float d0 = r2.x - c2.x, d1 = r2.y - c2.y;
        float acc = 0.0f;
        acc += d0 * d0;
        acc += d1 * d1;
        return acc;
    }
    const float* cw = cb + (size_t)e * ds;
    const float* r = rw + (e >> 4) * ds;
    float acc = 0.0f;
    for (int j = 0; j < ds; j++) {
        float diff = r[j] - cw[j];
        acc += diff * diff;
    }
    return acc;
}

// The quantised table of one list by one wave, its float entries computed
// from the residual and the codebooks in each of the two passes instead of
// kept.
__device__ inline void fs_build_qlut(const float* rw, const float* cb, int M, int ds, uint8_t* qlut,
                                     float& scale, float& base_offset) {
    fs_quantize_entries([&](int e) { return fs_lut_value(rw, cb, ds, e); }, qlut, M, scale, base_offset);
}

// Ascending bitonic sort of keys[0..n) by one wave (n a power of two).
__device__ inline void wave_bitonic_sort_keys(uint64_t* keys, int n) {
    const int lane = threadIdx.x & 63;
    for (int size = 2; size <= n; size <<= 1) {
        for (int stride = size >> 1; stride > 0; stride >>= 1) {
            wave_sync();
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
    wave_sync();
}

// Per-wave top-k buffer in LDS.
struct WaveTopk {
    uint64_t* keys;  // [buf]
    uint32_t* count; // wave counter
    uint32_t thr;    // accept fkey(dist) <= thr
    int buf, keep;

    __device__ void flush() {
        wave_sync();
        const int lane = threadIdx.x & 63;
        int n = (int)*count;
        int n2 = next_pow2(n > 0 ? n : 1);
        for (int i = n + lane; i < n2; i += 64) keys[i] = ~0ull;
        wave_bitonic_sort_keys(keys, n2);
        if (n >= keep) {
            thr = (uint32_t)(keys[keep - 1] >> 32);
            n = keep;
        }
        wave_sync();
        if (lane == 0) *count = (uint32_t)n;
        wave_sync();
    }

    // Push one candidate per lane (take may differ by lane); the insertion
    // index ids[pos] is read only for a candidate that passes the filter.
    __device__ void push(bool take, float dist, const uint32_t* __restrict__ ids, uint32_t pos) {
        uint32_t fk = fkey(dist);
        take = take && fk <= thr;
        uint64_t m = __ballot(take);
        if (m == 0) return;
        const uint32_t vidx = take ? ids[pos] : 0u;
        if ((int)*count > buf - 64) flush();
        take = take && fk <= thr;
        int slot = wave_append_slot(take, count);
        if (take) keys[slot] = ((uint64_t)fk << 32) | vidx;
        wave_sync();
    }
};

__host__ __device__ inline int fs_wave_buf(int keep) {
    int need = keep + 64;
    int b = 1;
    while (b < need) b <<= 1;
    return b;
}

__host__ __device__ inline size_t fs_align16(size_t x) { return (x + 15) & ~(size_t)15; }

// Probe slots staged in LDS per query; a wider probe reads each slot's list
// from global memory when its wave takes it.
#define FS_LDS_P 1024

__host__ __device__ inline size_t fs_lds_layout(int d, int M, int ds, int P, int wbuf, size_t* off) {
    if (P > FS_LDS_P) P = 0;
    size_t o = 0;
    off[0] = o; o = fs_align16(o + (size_t)d * 4);            // qs
    off[1] = o; o = fs_align16(o + (size_t)4 * d * 4);        // residual per wave
    off[2] = o; o = fs_align16(o + (fs_cb_in_lds(M, ds) ? (size_t)M * 16 * ds * 4 : 0));  // codebooks
    off[3] = o; o = fs_align16(o + (size_t)4 * 2 * M * 16);   // two byte LUTs per wave
    off[4] = o; o = fs_align16(o + (size_t)P * 4 * 2);        // lid, llen
    off[5] = o; o = fs_align16(o + (size_t)4 * wbuf * 8);     // wave buffers (contiguous)
    off[6] = o; o = fs_align16(o + 16 * 4);                   // counters
    return o;
}

// A list of a wave's block stream: its first stream block, blocks, entries,
// first packed block, quantisation and table slot.
struct FsList {
    uint32_t sst = 0, nb = 0, beg = 0, len = 0, pack = 0;
    float scale = 0.0f, base_offset = 0.0f;
    int slot = 0;
};

__global__ __launch_bounds__(256, 6) void fastscan_kernel(DevIndex ix, ScanArgs a, int wbuf) {
    extern __shared__ __align__(16) char smem[];
    const int q = blockIdx.x;
    if (q >= a.nq) return;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform: scalar
    const int d = ix.d, M = ix.M, ds = ix.ds, P = a.P;
    size_t off[7];
    fs_lds_layout(d, M, ds, P, wbuf, off);
    float* qs = (float*)(smem + off[0]);
    float* rw = (float*)(smem + off[1]) + wave * d;
    const bool cbl = fs_cb_in_lds(M, ds);
    float* cbs = (float*)(smem + off[2]);  // the codebooks when cbl
    uint8_t* qlut = (uint8_t*)(smem + off[3]) + wave * 2 * M * 16;  // [2][M * 16]
    const bool wide = P > FS_LDS_P;
    uint32_t* lid = (uint32_t*)(smem + off[4]);
    uint32_t* llen = lid + (wide ? 0 : P);
    uint64_t* allkeys = (uint64_t*)(smem + off[5]);
    uint32_t* cnt = (uint32_t*)(smem + off[6]);

    for (int j = tid; j < d; j += blockDim.x) qs[j] = a.qn[(size_t)q * d + j];
    for (int p = tid; p < (wide ? 0 : P); p += blockDim.x) {
        uint32_t l = a.probe[(size_t)q * P + p];
        bool ok = l < (uint32_t)ix.L;  // no such list: scanned as empty
        lid[p] = ok ? l : 0u;
        llen[p] = ok ? ix.offsets[l + 1] - ix.offsets[l] : 0u;
    }
    if (cbl)
        for (int i = tid; i < M * 16 * ds; i += blockDim.x) cbs[i] = ix.codebooks[i];
    if (tid < 4) cnt[tid] = 0;
    __syncthreads();

    WaveTopk tk;
    tk.keys = allkeys + (size_t)wave * wbuf;
    tk.count = cnt + wave;
    tk.thr = 0xffffffffu;
    tk.buf = wbuf;
    tk.keep = a.kout;
    uint32_t scanned = 0;

    // The wave's lists p = wave, wave + 4, ... in order.  Lists of 16 or more
    // entries form one stream of 32-entry blocks; each 16-block round takes the
    // next blocks of the stream from at most two lists (`prv`, `cur`), whose
    // quantised tables sit in the wave's two table slots.  A list's table is
    // built when the blocks ahead of the round run short and the older list's
    // blocks are all scanned (its slot is then free).  Shorter lists take the
    // exact float path as their table is built.
    // the packed blocks through a buffer resource: a lane's block offset in a
    // vector register once per round, each codebook's row offset a scalar
    const __amdgpu_buffer_rsrc_t prs = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint8_t*>(ix.packed), (short)0, (int)(ix.pack_off[ix.L] * 16u * (uint32_t)M), 0x00020000);
    FsList prv, cur;
    prv.slot = 0;
    cur.slot = 1;
    uint32_t s0 = 0;  // next stream block to scan
    int p = wave;     // next list to prepare
    for (;;) {
        while (p < P && cur.sst + cur.nb - s0 < 16 && prv.sst + prv.nb <= s0) {
            uint32_t l, len;
            if (wide) {
                const uint32_t g = a.probe[(size_t)q * P + p];
                const bool ok = g < (uint32_t)ix.L;  // no such list: scanned as empty
                l = ok ? g : 0u;
                len = ok ? ix.offsets[g + 1] - ix.offsets[g] : 0u;
            } else {
                l = lid[p];
                len = llen[p];
            }
            l = __builtin_amdgcn_readfirstlane(l);  // wave-uniform: scalar registers
            len = __builtin_amdgcn_readfirstlane(len);
            const int pp = p;
            p += 4;
            if (len == 0) continue;
            const uint32_t beg = ix.offsets[l];
            scanned += len;
            if (a.rres) {  // OPQ: R (q - c) from the rotation kernel (opq.rs:120-123)
                const float* rr = a.rres + ((size_t)q * P + pp) * d;
                for (int j = lane; j < d; j += 64) rw[j] = rr[j];
            } else {
                const float* c = ix.centroids + (size_t)l * d;
                for (int j = lane; j < d; j += 64) rw[j] = qs[j] - c[j];  // search.rs:1242-1245
            }
            wave_sync();
            if (len < 16) {
                // Exact float path: m-ordered sum of the float table (pq.rs:272-279).
                bool take = (uint32_t)lane < len;
                float dist = 0.0f;
                if (take) {
                    const uint8_t* row = ix.codes + (size_t)(beg + lane) * M;
                    if (cbl)
                        for (int m = 0; m < M; m++) dist += fs_lut_value(rw, cbs, ds, m * 16 + row[m]);
                    else
                        for (int m = 0; m < M; m++) dist += fs_lut_value(rw, ix.codebooks, ds, m * 16 + row[m]);
                }
                tk.push(take, dist, ix.list_ids, beg + lane);
                wave_sync();  // rw is rewritten for the next list
                continue;
            }
            // the older list is done: its slot takes the new list
            const int slot = prv.slot;
            prv = cur;
            cur.slot = slot;
            cur.sst = prv.sst + prv.nb;
            cur.nb = ix.pack_off[l + 1] - ix.pack_off[l];
            cur.beg = beg;
            cur.len = len;
            cur.pack = ix.pack_off[l];
            float sc, bo;
            if (cbl) fs_build_qlut(rw, cbs, M, ds, qlut + slot * M * 16, sc, bo);
            else fs_build_qlut(rw, ix.codebooks, M, ds, qlut + slot * M * 16, sc, bo);
            cur.scale = __uint_as_float(__builtin_amdgcn_readfirstlane(__float_as_uint(sc)));
            cur.base_offset = __uint_as_float(__builtin_amdgcn_readfirstlane(__float_as_uint(bo)));
            wave_sync();
        }
        const uint32_t s_end = cur.sst + cur.nb;
        if (s0 >= s_end) break;  // every list prepared and scanned
        // lane quad b scans stream block s0 + b of its list: 4 lanes x one code
        // dword of each codebook row (8 entries per lane)
        const uint32_t sb = s0 + (lane >> 2), w = lane & 3;
        const bool in_cur = sb >= cur.sst;
        const bool valid = sb < s_end;
        const uint32_t bl = valid ? sb - (in_cur ? cur.sst : prv.sst) : 0u;  // block within its list
        const uint32_t lbeg = in_cur ? cur.beg : prv.beg, llen_b = in_cur ? cur.len : prv.len;
        const float scale = in_cur ? cur.scale : prv.scale, base_offset = in_cur ? cur.base_offset : prv.base_offset;
        const uint32_t* qw = (const uint32_t*)(qlut + (in_cur ? cur.slot : prv.slot) * M * 16);
        uint32_t a0 = 0, a1 = 0, a2 = 0, a3 = 0;
        if (valid) {
            const uint32_t voff = ((in_cur ? cur.pack : prv.pack) + bl) * 16u * (uint32_t)M + 4u * w;
            // FS_CW codebooks' code words in flight at a time
            int m = 0;
            for (; m + FS_CW <= M; m += FS_CW) {
                uint32_t x[FS_CW];
#pragma unroll
                for (int u = 0; u < FS_CW; u++) x[u] = __builtin_amdgcn_raw_buffer_load_b32(prs, voff, (m + u) * 16, 0);
#pragma unroll
                for (int u = 0; u < FS_CW; u++)
                    fs_accumulate(x[u], qw[(m + u) * 4], qw[(m + u) * 4 + 1], qw[(m + u) * 4 + 2],
                                  qw[(m + u) * 4 + 3], a0, a1, a2, a3);
            }
            for (; m < M; m++)
                fs_accumulate(__builtin_amdgcn_raw_buffer_load_b32(prs, voff, m * 16, 0), qw[m * 4], qw[m * 4 + 1],
                              qw[m * 4 + 2], qw[m * 4 + 3], a0, a1, a2, a3);
        }
#pragma unroll
        for (int cc = 0; cc < 8; cc++) {
            const uint32_t vi = bl * 32 + (cc < 4 ? 4 * w + cc : 16 + 4 * w + (cc - 4));
            const bool take = valid && vi < llen_b;
            const float dist = take ? (float)fs_acc(cc, a0, a1, a2, a3) * scale + base_offset : 0.0f;
            tk.push(take, dist, ix.list_ids, lbeg + vi);
        }
        s0 = min(s0 + 16u, s_end);
        wave_sync();
    }
    tk.flush();
    // Pad each wave buffer past its kept prefix, then one block sort merges all.
    for (int i = (int)*tk.count + lane; i < wbuf; i += 64) tk.keys[i] = ~0ull;
    if (lane == 0) cnt[4 + wave] = scanned;
    __syncthreads();
    if (tid == 0) {
        uint32_t* st = a.qstat + (size_t)q * QSTAT_WORDS;
        st[0] = cnt[4] + cnt[5] + cnt[6] + cnt[7];
        st[1] = st[2] = st[3] = 0u;
    }
    block_bitonic_sort_keys(allkeys, 4 * wbuf);
    for (int j = tid; j < a.kout; j += blockDim.x) scan_emit(a, q, j, allkeys[j], allkeys[j] != ~0ull);
}

size_t fastscan_lds_bytes(const DevIndex& ix, const ScanArgs& a) {
    size_t off[7];
    return fs_lds_layout(ix.d, ix.M, ix.ds, a.P, fs_wave_buf(a.kout), off);
}

void launch_fastscan(const DevIndex& ix, const ScanArgs& a, hipStream_t s) {
    if (a.nq <= 0) return;
    size_t lds = fastscan_lds_bytes(ix, a);
    ensure_dyn_lds((const void*)fastscan_kernel, lds);
    hipLaunchKernelGGL(fastscan_kernel, dim3(a.nq), dim3(VGPU_BLOCK), lds, s, ix, a,
                       fs_wave_buf(a.kout));
}

// Test entry: one packed list, one wave quantises `lut` and scans every block.
__global__ void fastscan_test_kernel(const uint8_t* __restrict__ packed, int n, int M,
                                     const float* __restrict__ lut, float* __restrict__ out) {
    extern __shared__ __align__(16) char smem[];
    float* lutf = (float*)smem;
    uint8_t* qlut = (uint8_t*)(smem + fs_align16((size_t)M * 16 * 4));
    const int lane = threadIdx.x & 63;
    for (int e = lane; e < M * 16; e += 64) lutf[e] = lut[e];
    wave_sync();
    float scale, base_offset;
    fs_quantize(lutf, qlut, M, scale, base_offset);
    wave_sync();
    const uint32_t* qw = (const uint32_t*)qlut;
    const int nb = (n + 31) / 32;
    for (int b0 = 0; b0 < nb; b0 += 16) {
        const int b = b0 + (lane >> 2), w = lane & 3;
        uint32_t a0 = 0, a1 = 0, a2 = 0, a3 = 0;
        if (b < nb) {
            const uint32_t* src = (const uint32_t*)(packed + (size_t)b * 16 * M) + w;
            for (int m = 0; m < M; m++)
                fs_accumulate(src[m * 4], qw[m * 4], qw[m * 4 + 1], qw[m * 4 + 2], qw[m * 4 + 3], a0,
                              a1, a2, a3);
            for (int cc = 0; cc < 8; cc++) {
                const int vi = b * 32 + (cc < 4 ? 4 * w + cc : 16 + 4 * w + (cc - 4));
                if (vi < n) out[vi] = (float)fs_acc(cc, a0, a1, a2, a3) * scale + base_offset;
            }
        }
    }
}

void launch_fastscan_test(const uint8_t* packed, int n, int M, const float* lut, float* out,
                          hipStream_t s) {
    size_t lds = fs_align16((size_t)M * 16 * 4) + fs_align16((size_t)M * 16);
    ensure_dyn_lds((const void*)fastscan_test_kernel, lds);
    hipLaunchKernelGGL(fastscan_test_kernel, dim3(1), dim3(64), lds, s, packed, n, M, lut, out);
}

}  // namespace vgpu
