// File-backed IVF-PQ search: IVFPQFileSearcher (src/ivf_pq/search.rs:247-262,
// :1620-2041).  The routing metadata (centroids, codebooks, lists, doc ids)
// stays in memory and the centroids in HBM; the PQ codes and the raw vectors
// stay in the snapshot directory and are read per batch.
//
// One batch: the full index's coarse step gives every query's probe lists
// (search.rs:1904); the codes of the union of those lists are read from
// list_codes.bin (one positional read per list, list_offsets.bin giving the
// byte ranges; codes.bin row by row when the sidecar is absent, as
// search.rs:1953-1971 does) into a batch index of just those lists, which the
// in-HBM scan kernels search with the given probes.  The batch index numbers
// its vectors in ascending order of their index in the snapshot, so ties
// between equal distances resolve as in the full index.  A reranked search
// (search.rs:1835-1891) reads the raw vectors of the approximate candidates
// only (ascending offsets, :1871) and rescores them on the GPU.
#include <fcntl.h>
#include <unistd.h>

#include <algorithm>
#include <cmath>
#include <cstring>

#include "vgpu_launch.h"
#include "vgpu_runtime.h"

namespace vgpu {

namespace {

void read_at(int fd, uint64_t off, void* dst, size_t bytes, const char* what) {
    uint8_t* p = static_cast<uint8_t*>(dst);
    while (bytes) {
        const ssize_t r = pread(fd, p, bytes, (off_t)off);
        if (r <= 0) throw Error(VGPU_ERR_INVALID_PARAMETER, std::string("short read of ") + what);
        p += r;
        off += (uint64_t)r;
        bytes -= (size_t)r;
    }
}

int open_file(const std::string& path, bool required) {
    const int fd = ::open(path.c_str(), O_RDONLY | O_CLOEXEC);
    if (fd < 0 && required) throw Error(VGPU_ERR_INVALID_PARAMETER, "cannot open " + path);
    return fd;
}

uint64_t file_size(int fd) {
    const off_t e = lseek(fd, 0, SEEK_END);
    return e < 0 ? 0 : (uint64_t)e;
}

}  // namespace

UniqueFd::~UniqueFd() {
    if (v >= 0) ::close(v);
}

FileIvfpq::FileIvfpq(size_t dim, const vgpu_ivfpq_params& p, const float* cent, size_t Lc, const float* cb,
                     size_t Kc, const uint64_t* off, const uint32_t* lids, const uint32_t* dids, size_t nv,
                     const float* rot, const std::string& directory, bool raw_present)
    : d(dim), params(p), dir(directory) {
    // Host-side checks and file opens first, so a malformed snapshot is
    // reported before any device work.
    if (!dim || !p.num_codebooks || dim % p.num_codebooks)
        throw Error(VGPU_ERR_INVALID_CONFIG, "dimension must be divisible by num_codebooks");
    if (!Lc || !Kc || Kc > 256)
        throw Error(VGPU_ERR_INVALID_CONFIG, "need num_centroids > 0 and 1 <= codebook_size <= 256");
    L = Lc;
    K = Kc;
    n = nv;
    M = p.num_codebooks;
    if (nv && (!lids || !dids)) throw Error(VGPU_ERR_INVALID_PARAMETER, "null argument");
    if (off[0] != 0 || off[L] != nv)
        throw Error(VGPU_ERR_INVALID_PARAMETER, "list_offsets must start at 0 and end at num_vectors");
    offsets.assign(off, off + L + 1);
    list_ids.assign(lids, lids + nv);
    doc_ids.assign(dids, dids + nv);
    centroids.assign(cent, cent + L * d);
    codebooks.assign(cb, cb + M * K * (d / M));
    for (size_t l = 0; l < L; l++)
        if (offsets[l + 1] < offsets[l])
            throw Error(VGPU_ERR_INVALID_PARAMETER, "list_offsets must be non-decreasing");
    {
        std::vector<uint8_t> seen(nv, 0);  // each vector in exactly one list position
        for (size_t i = 0; i < nv; i++) {
            if (list_ids[i] >= nv) throw Error(VGPU_ERR_INVALID_PARAMETER, "list id beyond num_vectors");
            if (seen[list_ids[i]]++)
                throw Error(VGPU_ERR_INVALID_PARAMETER, "list_ids must be a permutation of 0..num_vectors");
        }
    }
    // search.rs:1707-1735: list_codes.bin + list_offsets.bin when present
    // (both or neither), codes.bin otherwise; raw_vectors.bin for rerank.
    fd_codes.v = open_file(dir + "/codes.bin", true);
    if (file_size(fd_codes.v) != (uint64_t)nv * M)
        throw Error(VGPU_ERR_INVALID_PARAMETER, "codes.bin size does not match num_vectors * num_codebooks");
    UniqueFd fo;
    fo.v = open_file(dir + "/list_offsets.bin", false);
    fd_list_codes.v = open_file(dir + "/list_codes.bin", false);
    if ((fo.v < 0) != (fd_list_codes.v < 0))
        throw Error(VGPU_ERR_INVALID_PARAMETER,
                    "partial IVF-PQ list-code sidecar: expected both list_offsets.bin and list_codes.bin");
    if (fo.v >= 0) {
        const size_t nl = p.num_clusters;
        if (nl < L || file_size(fo.v) != (uint64_t)(nl + 1) * 8)
            throw Error(VGPU_ERR_INVALID_PARAMETER, "list_offsets.bin size does not match num_clusters");
        lc_offsets.resize(nl + 1);
        read_at(fo.v, 0, lc_offsets.data(), (nl + 1) * 8, "list_offsets.bin");
        // file_storage.rs validate_list_code_offsets: monotone, whole rows,
        // ending at the codes length, and each list's row count
        if (lc_offsets[0] != 0 || lc_offsets[nl] != (uint64_t)nv * M)
            throw Error(VGPU_ERR_INVALID_PARAMETER, "list_offsets.bin does not span the codes");
        for (size_t l = 0; l < nl; l++) {
            const uint64_t len = l < L ? offsets[l + 1] - offsets[l] : 0;
            if (lc_offsets[l + 1] < lc_offsets[l] || lc_offsets[l + 1] - lc_offsets[l] != len * M)
                throw Error(VGPU_ERR_INVALID_PARAMETER, "list_offsets.bin disagrees with the lists");
        }
        if (file_size(fd_list_codes.v) != (uint64_t)nv * M)
            throw Error(VGPU_ERR_INVALID_PARAMETER, "list_codes.bin size does not match the codes");
    }
    if (raw_present) {
        fd_raw.v = open_file(dir + "/raw_vectors.bin", true);
        if (file_size(fd_raw.v) != (uint64_t)nv * d * 4)
            throw Error(VGPU_ERR_INVALID_PARAMETER, "raw_vectors.bin size does not match the vectors");
    }
    // The coarse step only: every list empty, so nothing but the centroids,
    // codebooks and their device copies is held.
    meta = std::make_unique<IvfpqIndex>(dim, p);
    batch = std::make_unique<IvfpqIndex>(dim, p);
    if (rot) {
        meta->set_rotation(rot);
        batch->set_rotation(rot);
    }
    const std::vector<uint64_t> zero(L + 1, 0);
    meta->load(cent, Lc, cb, Kc, zero.data(), nullptr, nullptr, nullptr, nullptr, 0);
    VGPU_HIP(hipStreamCreateWithFlags(&stream, hipStreamNonBlocking));
}

FileIvfpq::~FileIvfpq() {
    if (stream) (void)hipStreamDestroy(stream);
}

// The batch index: the lists of `uni` (ascending list ids) with their codes
// read from the snapshot; vectors numbered in ascending snapshot order.
void FileIvfpq::load_batch(const std::vector<uint32_t>& uni, std::vector<uint32_t>& members) {
    members.clear();
    for (uint32_t l : uni)
        members.insert(members.end(), list_ids.begin() + (ptrdiff_t)offsets[l],
                       list_ids.begin() + (ptrdiff_t)offsets[l + 1]);
    std::sort(members.begin(), members.end());
    const size_t nb = members.size();
    auto rank = [&](uint32_t g) {
        return (uint32_t)(std::lower_bound(members.begin(), members.end(), g) - members.begin());
    };
    std::vector<uint64_t> boff(uni.size() + 1, 0);
    std::vector<uint32_t> blids(nb);
    std::vector<uint8_t> bcodes(std::max<size_t>(nb * M, 1));
    std::vector<float> bcent(uni.size() * d);
    std::vector<uint8_t> buf;
    for (size_t u = 0; u < uni.size(); u++) {
        const uint32_t l = uni[u];
        const size_t beg = offsets[l], len = offsets[l + 1] - beg;
        std::memcpy(&bcent[u * d], &centroids[(size_t)l * d], d * sizeof(float));
        boff[u + 1] = boff[u] + len;
        if (len == 0) continue;
        if (fd_list_codes.v >= 0) {  // read_list_codes_for_cluster (file_storage.rs:119-155)
            buf.resize(len * M);
            read_at(fd_list_codes.v, lc_offsets[l], buf.data(), len * M, "list_codes.bin");
            io_reads++;
            io_bytes += len * M;
            for (size_t i = 0; i < len; i++) {
                const uint32_t r = rank(list_ids[beg + i]);
                blids[boff[u] + i] = r;
                std::memcpy(&bcodes[(size_t)r * M], &buf[i * M], M);
            }
        } else {  // append_codes_for_ids (file_storage.rs:98-117): row by row
            for (size_t i = 0; i < len; i++) {
                const uint32_t g = list_ids[beg + i], r = rank(g);
                blids[boff[u] + i] = r;
                read_at(fd_codes.v, (uint64_t)g * M, &bcodes[(size_t)r * M], M, "codes.bin");
                io_reads++;
                io_bytes += M;
            }
        }
    }
    batch->load(bcent.data(), uni.size(), codebooks.data(), K, boff.data(), blids.data(), bcodes.data(),
                nullptr, nullptr, nb);
}

void FileIvfpq::search(const float* q, size_t nq, size_t k, size_t nprobe, size_t pool, int64_t* ids,
                       float* dists, vgpu_file_diagnostics* diag) {
    for (size_t i = 0; i < nq * d; i++)
        if (!std::isfinite(q[i])) throw Error(VGPU_ERR_INVALID_PARAMETER, "query contains a non-finite value");
    if (pool && fd_raw.v < 0)
        throw Error(VGPU_ERR_UNSUPPORTED, "search_reranked without raw vectors");
    io_bytes = io_reads = 0;
    for (size_t i = 0; i < nq * k; i++) {
        ids[i] = -1;
        dists[i] = INFINITY;
    }
    if (diag) std::memset(diag, 0, nq * sizeof(vgpu_file_diagnostics));
    const size_t P = std::min(nprobe ? nprobe : params.nprobe, L);
    if (nq == 0 || k == 0 || P == 0) return;
    // the full index's probe lists, then the batch index over their union
    std::vector<uint32_t> probes(nq * P);
    meta->probe_host(q, nq, P, probes.data());
    std::vector<uint32_t> uni(probes);
    std::sort(uni.begin(), uni.end());
    uni.erase(std::unique(uni.begin(), uni.end()), uni.end());
    std::vector<uint32_t> members;
    load_batch(uni, members);
    for (auto& l : probes) l = (uint32_t)(std::lower_bound(uni.begin(), uni.end(), l) - uni.begin());
    const size_t kk = pool ? std::max(pool, k) : k;  // search.rs:1853
    std::vector<int64_t> bids(nq * kk);
    std::vector<float> bd(nq * kk);
    batch->search_host_probed(q, nq, P, probes.data(), kk, bids.data(), bd.data());
    for (size_t qi = 0; qi < nq && diag; qi++) {  // search.rs:1904-1980
        vgpu_file_diagnostics& g = diag[qi];
        g.probed_lists = P;
        for (size_t p = 0; p < P; p++) {
            const uint32_t u = probes[qi * P + p];
            const uint64_t len = batch->offsets[u + 1] - batch->offsets[u];
            g.scanned_vectors += len;
            g.code_bytes += len * M;
            g.code_reads += (len >= 16 && fd_list_codes.v >= 0) ? 1 : len;
        }
        size_t found = 0;
        while (found < kk && bids[qi * kk + found] >= 0) found++;
        g.retained_candidates = found;
    }
    if (!pool) {
        for (size_t qi = 0; qi < nq; qi++)
            for (size_t j = 0; j < k; j++) {
                const int64_t b = bids[qi * kk + j];
                if (b < 0) continue;
                ids[qi * k + j] = doc_ids[members[(size_t)b]];
                dists[qi * k + j] = bd[qi * kk + j];
            }
        return;
    }
    // Rerank: the raw vectors of the distinct candidates, ascending offsets.
    std::vector<uint32_t> cand;
    for (int64_t b : bids)
        if (b >= 0) cand.push_back(members[(size_t)b]);
    std::sort(cand.begin(), cand.end());
    cand.erase(std::unique(cand.begin(), cand.end()), cand.end());
    std::vector<float> vecs(std::max<size_t>(cand.size(), 1) * d);
    for (size_t i = 0; i < cand.size(); i++) {
        read_at(fd_raw.v, (uint64_t)cand[i] * d * 4, &vecs[i * d], d * 4, "raw_vectors.bin");
        io_reads++;
        io_bytes += d * 4;
    }
    std::vector<uint32_t> rows(nq * kk, 0xffffffffu);
    for (size_t i = 0; i < nq * kk; i++)
        if (bids[i] >= 0)
            rows[i] = (uint32_t)(std::lower_bound(cand.begin(), cand.end(), members[(size_t)bids[i]]) -
                                 cand.begin());
    for (size_t qi = 0; qi < nq && diag; qi++) {
        diag[qi].raw_vector_reads = diag[qi].retained_candidates;
        diag[qi].raw_vector_bytes = diag[qi].retained_candidates * d * 4;
        diag[qi].reranked_candidates = diag[qi].retained_candidates;
    }
    d_vecs.upload(vecs.data(), vecs.size(), stream);
    d_rows.upload(rows.data(), rows.size(), stream);
    d_q.upload(q, nq * d, stream);
    d_qn.reserve(nq * d);
    d_outrow.reserve(nq * k);
    d_outd.reserve(nq * k);
    std::vector<uint32_t> orow(nq * k);
    std::vector<float> od(nq * k);
    launch_normalize(d_q.p, d_qn.p, nullptr, (int)nq, (int)d, stream);  // search.rs:1865
    launch_rerank_vectors(d_vecs.p, (int)d, d_qn.p, (int)nq, d_rows.p, (int)kk, (int)k, d_outrow.p, d_outd.p,
                          stream);
    VGPU_HIP(hipGetLastError());
    VGPU_HIP(hipMemcpyAsync(orow.data(), d_outrow.p, nq * k * 4, hipMemcpyDeviceToHost, stream));
    VGPU_HIP(hipMemcpyAsync(od.data(), d_outd.p, nq * k * 4, hipMemcpyDeviceToHost, stream));
    VGPU_HIP(hipStreamSynchronize(stream));
    for (size_t i = 0; i < nq * k; i++) {
        if (orow[i] == 0xffffffffu) continue;
        if (orow[i] >= cand.size()) throw Error(VGPU_ERR_DEVICE, "rerank returned a row out of range");
        ids[i] = doc_ids[cand[orow[i]]];
        dists[i] = od[i];
    }
}

}  // namespace vgpu
