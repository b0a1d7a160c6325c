// Direct-to-device upload of byte ranges of a file (the load path of the
// device image).  Host code only: reader threads pread fixed-size pieces
// into pinned staging buffers and each piece goes to its device destination
// by hipMemcpyAsync on the thread's own stream, while the thread reads its
// next piece into its second buffer.  The file is never mapped and nothing
// is decoded or re-indexed on the host.
#include "../../include/cbq_hip.h"

#include <errno.h>
#include <fcntl.h>
#include <sys/stat.h>
#include <stdio.h>
#include <string.h>
#include <unistd.h>

#include <atomic>
#include <thread>
#include <vector>

namespace {

struct Piece {
    int64_t file_offset;
    int64_t nbytes;
    char *dst;
};

struct Worker {
    hipStream_t stream = nullptr;
    hipEvent_t done[2] = {nullptr, nullptr};
    char *buf[2] = {nullptr, nullptr};
};

// Fills buf with exactly n bytes from fd at offset off (pread may return
// short counts).  False on an I/O error or end of file.
bool read_full(int fd, char *buf, int64_t n, int64_t off)
{
    while (n > 0) {
        const ssize_t r = pread(fd, buf, (size_t)n, (off_t)off);
        if (r < 0 && errno == EINTR) continue;
        if (r <= 0) return false;
        buf += r;
        n -= r;
        off += r;
    }
    return true;
}

}  // namespace

extern "C" int cbq_file_upload(const char *path, const cbq_upload_part *parts, int n_parts,
                               size_t chunk_bytes, int n_threads)
{
    if (!path || n_parts < 0 || (n_parts > 0 && !parts) || chunk_bytes < 4096 ||
        chunk_bytes > ((size_t)1 << 30) || n_threads < 1 || n_threads > 64)
        return CK_ERR_ARG;
    std::vector<Piece> pieces;
    for (int i = 0; i < n_parts; i++) {
        const cbq_upload_part &p = parts[i];
        if (p.file_offset < 0 || p.nbytes < 0 || (p.nbytes > 0 && !p.dst)) return CK_ERR_ARG;
        for (int64_t o = 0; o < p.nbytes; o += (int64_t)chunk_bytes) {
            const int64_t n = p.nbytes - o < (int64_t)chunk_bytes ? p.nbytes - o
                                                                  : (int64_t)chunk_bytes;
            pieces.push_back({p.file_offset + o, n, (char *)p.dst + o});
        }
    }
    if (pieces.empty()) return CK_SUCCESS;
    const int fd = open(path, O_RDONLY | O_CLOEXEC);
    if (fd < 0) {
        fprintf(stderr, "cbq_file_upload: cannot open %s: %s\n", path, strerror(errno));
        return CK_ERR_ARG;
    }
    // every range inside the file, checked before any HIP call
    struct stat st;
    if (fstat(fd, &st) != 0) {
        fprintf(stderr, "cbq_file_upload: cannot stat %s: %s\n", path, strerror(errno));
        close(fd);
        return CK_ERR_ARG;
    }
    for (int i = 0; i < n_parts; i++)
        if (parts[i].file_offset > (int64_t)st.st_size ||
            parts[i].nbytes > (int64_t)st.st_size - parts[i].file_offset) {
            fprintf(stderr, "cbq_file_upload: range [%lld, +%lld) past the end of %s (%lld bytes)\n",
                    (long long)parts[i].file_offset, (long long)parts[i].nbytes, path,
                    (long long)st.st_size);
            close(fd);
            return CK_ERR_ARG;
        }
    const int nw = n_threads < (int)pieces.size() ? n_threads : (int)pieces.size();
    std::vector<Worker> w(nw);
    hipError_t herr = hipSuccess;
    for (int t = 0; t < nw && herr == hipSuccess; t++) {
        herr = hipStreamCreateWithFlags(&w[t].stream, hipStreamNonBlocking);
        for (int b = 0; b < 2 && herr == hipSuccess; b++) {
            herr = hipHostMalloc((void **)&w[t].buf[b], chunk_bytes, hipHostMallocDefault);
            if (herr == hipSuccess)
                herr = hipEventCreateWithFlags(&w[t].done[b], hipEventDisableTiming);
        }
    }
    std::atomic<size_t> next{0};
    std::atomic<int> status{herr == hipSuccess ? CK_SUCCESS : CK_ERR_HIP};
    if (herr != hipSuccess)
        fprintf(stderr, "cbq_file_upload: staging set-up: %s\n", hipGetErrorString(herr));
    auto run = [&](int t) {
        Worker &me = w[t];
        int slot = 0;
        bool used[2] = {false, false};
        for (;;) {
            if (status.load() != CK_SUCCESS) return;
            const size_t i = next.fetch_add(1);
            if (i >= pieces.size()) return;
            const Piece &pc = pieces[i];
            // the buffer's previous copy must have left it before it is refilled
            if (used[slot]) {
                const hipError_t e = hipEventSynchronize(me.done[slot]);
                if (e != hipSuccess) {
                    fprintf(stderr, "cbq_file_upload: %s\n", hipGetErrorString(e));
                    status.store(CK_ERR_HIP);
                    return;
                }
            }
            if (!read_full(fd, me.buf[slot], pc.nbytes, pc.file_offset)) {
                fprintf(stderr, "cbq_file_upload: short read of %s at %lld (+%lld bytes)\n",
                        path, (long long)pc.file_offset, (long long)pc.nbytes);
                status.store(CK_ERR_ARG);
                return;
            }
            hipError_t e = hipMemcpyAsync(pc.dst, me.buf[slot], (size_t)pc.nbytes,
                                          hipMemcpyHostToDevice, me.stream);
            if (e == hipSuccess) e = hipEventRecord(me.done[slot], me.stream);
            if (e != hipSuccess) {
                fprintf(stderr, "cbq_file_upload: %s\n", hipGetErrorString(e));
                status.store(CK_ERR_HIP);
                return;
            }
            used[slot] = true;
            slot ^= 1;
        }
    };
    if (status.load() == CK_SUCCESS) {
        std::vector<std::thread> th;
        for (int t = 1; t < nw; t++) th.emplace_back(run, t);
        run(0);
        for (auto &x : th) x.join();
    }
    // every issued copy finishes before its staging buffer is freed
    for (int t = 0; t < nw; t++) {
        if (w[t].stream) {
            const hipError_t e = hipStreamSynchronize(w[t].stream);
            if (e != hipSuccess && status.load() == CK_SUCCESS) {
                fprintf(stderr, "cbq_file_upload: %s\n", hipGetErrorString(e));
                status.store(CK_ERR_HIP);
            }
        }
        for (int b = 0; b < 2; b++) {
            if (w[t].done[b]) (void)hipEventDestroy(w[t].done[b]);
            if (w[t].buf[b]) (void)hipHostFree(w[t].buf[b]);
        }
        if (w[t].stream) (void)hipStreamDestroy(w[t].stream);
    }
    close(fd);
    return status.load();
}

// Host buffer -> fresh device allocation (synchronous copy); nullptr on any
// failure, with nothing left allocated.
static void *upload_bytes(const void *host, size_t nbytes, const char *what)
{
    if (!host || nbytes == 0) return nullptr;
    void *dev = nullptr;
    hipError_t e = hipMalloc(&dev, nbytes);
    if (e != hipSuccess) {
        fprintf(stderr, "%s: hipMalloc(%zu): %s\n", what, nbytes, hipGetErrorString(e));
        return nullptr;
    }
    e = hipMemcpy(dev, host, nbytes, hipMemcpyHostToDevice);
    if (e != hipSuccess) {
        fprintf(stderr, "%s: hipMemcpy: %s\n", what, hipGetErrorString(e));
        (void)hipFree(dev);
        return nullptr;
    }
    return dev;
}

extern "C" uint8_t *ck_upload_packed(const uint8_t *host_packed, size_t nbytes)
{
    return (uint8_t *)upload_bytes(host_packed, nbytes, "ck_upload_packed");
}

extern "C" float *ck_upload_codebook(const float *host_codebook, int C)
{
    if (C <= 0) return nullptr;
    return (float *)upload_bytes(host_codebook, (size_t)C * sizeof(float), "ck_upload_codebook");
}
