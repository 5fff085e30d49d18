// Loading a model's packed weights into HBM once (the weight-residency row of the path).
//
// The reference streams every projection's packed bytes to the GPU on every call: the host
// wrappers copy the whole weight per call (src/kernels/dequantize.hip:729-762 and siblings), and
// the device-resident layer still copies each projection through one staging buffer before its
// kernel (project_on_device, src/kernels/attention.hip:572-599), reading the file through a
// page-cache-managed mmap (WeightStreamer, src/weight_loader.py:99-187).  On MI355X a whole
// quantized model fits in the 288 GB of HBM, so the weights are read from the file once, with
// the read of one chunk overlapping the host -> device copy of the previous one:
//   * several reader threads pread() disjoint pieces of a chunk into a pinned staging buffer;
//   * the chunk is then copied to its device destination with hipMemcpyAsync on the caller's
//     stream, and an event marks when the buffer is free again;
//   * `depth` staging buffers rotate, so reading chunk c overlaps the copies of chunks
//     c - depth + 1 .. c - 1.
// The pinned staging buffers are kept between calls (grow-only) and freed by
// qmm_release_workspace().  qmm_read_file() is the same reader with host destinations and no
// staging (no GPU needed).
#include <fcntl.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <atomic>
#include <cerrno>
#include <cstring>
#include <condition_variable>
#include <functional>
#include <mutex>
#include <string>
#include <thread>
#include <vector>

#include "qmm_internal.h"

namespace qmm {
namespace {

// Fork-join pool: run(n, f) calls f(i) for i < n on the pool's threads and returns when all are
// done.  Task indices are taken under the mutex (tasks are multi-megabyte reads), so a worker
// always runs the current job with one of its own indices.
class Pool {
public:
    explicit Pool(int threads) {
        for (int t = 0; t < threads; ++t) workers_.emplace_back([this] { loop(); });
    }
    ~Pool() {
        {
            std::lock_guard<std::mutex> lk(mu_);
            stop_ = true;
        }
        cv_.notify_all();
        for (auto& w : workers_) w.join();
    }
    void run(int n, const std::function<void(int)>& f) {
        std::unique_lock<std::mutex> lk(mu_);
        job_ = &f;
        n_ = n;
        next_ = 0;
        pending_ = n;
        ++gen_;
        cv_.notify_all();
        done_cv_.wait(lk, [this] { return pending_ == 0; });
        job_ = nullptr;
        n_ = 0;
    }

private:
    void loop() {
        uint64_t seen = 0;
        std::unique_lock<std::mutex> lk(mu_);
        for (;;) {
            cv_.wait(lk, [&] { return stop_ || gen_ != seen; });
            if (stop_) return;
            seen = gen_;
            while (next_ < n_) {
                const int i = next_++;
                const std::function<void(int)>* job = job_;
                lk.unlock();
                (*job)(i);
                lk.lock();
                if (--pending_ == 0) done_cv_.notify_all();
            }
        }
    }
    std::vector<std::thread> workers_;
    std::mutex mu_;
    std::condition_variable cv_, done_cv_;
    const std::function<void(int)>* job_ = nullptr;
    int n_ = 0, next_ = 0, pending_ = 0;
    uint64_t gen_ = 0;
    bool stop_ = false;
};

struct File {
    int fd = -1;
    ~File() {
        if (fd >= 0) close(fd);
    }
};

constexpr int64_t kMinChunk = int64_t{4} << 20;

// Bytes per pread task: about two tasks per thread for `total` bytes, in [256 KiB, 4 MiB] and a
// multiple of 64 KiB, so every reader thread has work even for one staging chunk.
int64_t piece_bytes(int64_t total, int threads) {
    const int64_t want = (total / (2 * static_cast<int64_t>(threads)) + 0xFFFF) & ~int64_t{0xFFFF};
    return std::max<int64_t>(int64_t{256} << 10, std::min<int64_t>(want, int64_t{4} << 20));
}

// pread [off, off + n) into dst, whole; false (errno kept) on error or early end of file.
bool pread_all(int fd, char* dst, int64_t n, int64_t off) {
    while (n > 0) {
        const ssize_t r = pread(fd, dst, static_cast<size_t>(std::min<int64_t>(n, int64_t{1} << 30)), off);
        if (r < 0 && errno == EINTR) continue;
        if (r == 0) errno = 0;  // end of file
        if (r <= 0) return false;
        dst += r;
        off += r;
        n -= r;
    }
    return true;
}

// The listed spans, each (file offset, bytes, destination), read in parallel in pieces of
// `piece` bytes.
struct Span {
    int64_t off, bytes;
    char* dst;
};

UploadStatus read_spans(Pool& pool, int fd, const std::vector<Span>& spans, int64_t piece) {
    std::vector<std::pair<int, int64_t>> tasks;  // (span, piece start within the span)
    for (int s = 0; s < static_cast<int>(spans.size()); ++s)
        for (int64_t p = 0; p < spans[s].bytes; p += piece) tasks.emplace_back(s, p);
    std::atomic<int> bad{-1};
    std::atomic<int> bad_errno{0};
    pool.run(static_cast<int>(tasks.size()), [&](int i) {
        const Span& sp = spans[tasks[i].first];
        const int64_t p = tasks[i].second;
        const int64_t n = std::min(piece, sp.bytes - p);
        if (!pread_all(fd, sp.dst + p, n, sp.off + p)) {
            int expect = -1;
            if (bad.compare_exchange_strong(expect, i)) bad_errno.store(errno);
        }
    });
    if (bad.load() >= 0) {
        const Span& sp = spans[tasks[bad.load()].first];
        return {QMM_ERR_IO, "read of file bytes [" + std::to_string(sp.off) + ", " + std::to_string(sp.off + sp.bytes) +
                                ") failed" + (bad_errno.load() ? std::string(": ") + strerror(bad_errno.load()) : ": end of file")};
    }
    return {QMM_OK, ""};
}

UploadStatus open_checked(const char* path, const FileRange* ranges, int count, File& f) {
    if (path == nullptr) return {QMM_ERR_INVALID_ARGUMENT, "path must be non-null."};
    if (count < 0 || (count > 0 && ranges == nullptr))
        return {QMM_ERR_INVALID_ARGUMENT, "ranges must hold count >= 0 entries."};
    f.fd = open(path, O_RDONLY | O_CLOEXEC);
    if (f.fd < 0) return {QMM_ERR_IO, std::string("cannot open ") + path + ": " + strerror(errno)};
    struct stat st;
    if (fstat(f.fd, &st) != 0) return {QMM_ERR_IO, std::string("cannot stat ") + path + ": " + strerror(errno)};
    for (int i = 0; i < count; ++i) {
        const FileRange& r = ranges[i];
        if (r.offset < 0 || r.bytes < 0 || r.offset > st.st_size || r.bytes > st.st_size - r.offset)
            return {QMM_ERR_INVALID_ARGUMENT, "range " + std::to_string(i) + " [" + std::to_string(r.offset) + ", " +
                                                  std::to_string(r.offset + r.bytes) + ") exceeds the file size " +
                                                  std::to_string(static_cast<long long>(st.st_size)) + "."};
        if (r.bytes > 0 && r.dst == nullptr)
            return {QMM_ERR_INVALID_ARGUMENT, "range " + std::to_string(i) + " has a null destination."};
    }
    return {QMM_OK, ""};
}

int clamp_threads(int threads) { return std::max(1, std::min(threads, 64)); }

// Pinned staging buffers kept between calls (allocating gigabytes of pinned memory costs more
// than moving them): grow-only, freed by release_upload_staging().  One load runs at a time.
struct Staging {
    std::mutex mu;
    std::vector<char*> bufs;
    int64_t cap = 0;
};
Staging g_staging;

// Requires g_staging.mu held.  At least `depth` buffers of at least `bytes`.
hipError_t staging_ensure(int depth, int64_t bytes) {
    if (g_staging.cap >= bytes && static_cast<int>(g_staging.bufs.size()) >= depth) return hipSuccess;
    for (char* b : g_staging.bufs) (void)hipHostFree(b);
    g_staging.bufs.clear();
    g_staging.cap = 0;
    for (int i = 0; i < depth; ++i) {
        char* b = nullptr;
        hipError_t e = hipHostMalloc(reinterpret_cast<void**>(&b), static_cast<size_t>(bytes), hipHostMallocDefault);
        if (e != hipSuccess) {
            for (char* x : g_staging.bufs) (void)hipHostFree(x);
            g_staging.bufs.clear();
            return e;
        }
        g_staging.bufs.push_back(b);
    }
    g_staging.cap = bytes;
    return hipSuccess;
}

}  // namespace

void release_upload_staging() {
    std::lock_guard<std::mutex> lk(g_staging.mu);
    for (char* b : g_staging.bufs) (void)hipHostFree(b);
    g_staging.bufs.clear();
    g_staging.cap = 0;
}

UploadStatus read_file_ranges(const char* path, const FileRange* ranges, int count, int threads) {
    File f;
    UploadStatus st = open_checked(path, ranges, count, f);
    if (st.code != QMM_OK) return st;
    std::vector<Span> spans;
    int64_t total = 0;
    for (int i = 0; i < count; ++i)
        if (ranges[i].bytes > 0) {
            spans.push_back({ranges[i].offset, ranges[i].bytes, static_cast<char*>(ranges[i].dst)});
            total += ranges[i].bytes;
        }
    const int nt = clamp_threads(threads);
    Pool pool(nt);
    return read_spans(pool, f.fd, spans, piece_bytes(total, nt));
}

UploadStatus upload_file_ranges(const char* path, const FileRange* ranges, int count, int64_t chunk_bytes, int depth,
                                int threads, hipStream_t stream) {
    File f;
    UploadStatus st = open_checked(path, ranges, count, f);
    if (st.code != QMM_OK) return st;
    if (chunk_bytes < kMinChunk || chunk_bytes > (int64_t{1} << 32))
        return {QMM_ERR_INVALID_ARGUMENT, "chunk_bytes must be in [4 MiB, 4 GiB]."};
    if (depth < 2 || depth > 8) return {QMM_ERR_INVALID_ARGUMENT, "depth must be in [2, 8]."};

    // chunks: consecutive pieces of the ranges, each at most chunk_bytes (several small ranges
    // share a chunk)
    struct Part {
        int64_t off, bytes;
        char* dst;       // device destination
        int64_t at;      // offset inside the staging buffer
    };
    std::vector<std::vector<Part>> chunks(1);
    int64_t fill = 0;
    for (int i = 0; i < count; ++i) {
        int64_t done = 0;
        while (done < ranges[i].bytes) {
            if (fill == chunk_bytes) {
                chunks.emplace_back();
                fill = 0;
            }
            const int64_t n = std::min(ranges[i].bytes - done, chunk_bytes - fill);
            chunks.back().push_back({ranges[i].offset + done, n, static_cast<char*>(ranges[i].dst) + done, fill});
            fill += n;
            done += n;
        }
    }
    if (chunks.back().empty()) chunks.pop_back();
    if (chunks.empty()) return {QMM_OK, ""};

    const int nbuf = std::min<int>(depth, static_cast<int>(chunks.size()));
    std::lock_guard<std::mutex> staging_lock(g_staging.mu);
    hipError_t se = staging_ensure(nbuf, chunk_bytes);
    if (se != hipSuccess) return {QMM_ERR_HIP, std::string("hipHostMalloc (staging): ") + hipGetErrorString(se)};
    const std::vector<char*>& buf = g_staging.bufs;
    std::vector<hipEvent_t> ev(nbuf, nullptr);
    auto cleanup = [&](UploadStatus s) {
        // every copy out of a staging buffer must finish before the buffer is reused
        hipError_t e = hipStreamSynchronize(stream);
        if (e != hipSuccess && s.code == QMM_OK) s = {QMM_ERR_HIP, std::string("hipStreamSynchronize: ") + hipGetErrorString(e)};
        for (int b = 0; b < nbuf; ++b)
            if (ev[b]) (void)hipEventDestroy(ev[b]);
        return s;
    };
    for (int b = 0; b < nbuf; ++b) {
        hipError_t e = hipEventCreateWithFlags(&ev[b], hipEventDisableTiming);
        if (e != hipSuccess) {
            ev[b] = nullptr;
            return cleanup({QMM_ERR_HIP, std::string("hipEventCreate: ") + hipGetErrorString(e)});
        }
    }
    const int nt = clamp_threads(threads);
    const int64_t piece = piece_bytes(chunk_bytes, nt);
    Pool pool(nt);
    for (size_t c = 0; c < chunks.size(); ++c) {
        const int b = static_cast<int>(c % nbuf);
        hipError_t e;
        if (c >= static_cast<size_t>(nbuf) && (e = hipEventSynchronize(ev[b])) != hipSuccess)
            return cleanup({QMM_ERR_HIP, std::string("hipEventSynchronize: ") + hipGetErrorString(e)});
        std::vector<Span> spans;
        for (const Part& p : chunks[c]) spans.push_back({p.off, p.bytes, buf[b] + p.at});
        UploadStatus rs = read_spans(pool, f.fd, spans, piece);
        if (rs.code != QMM_OK) return cleanup(rs);
        for (const Part& p : chunks[c]) {
            if ((e = hipMemcpyAsync(p.dst, buf[b] + p.at, static_cast<size_t>(p.bytes), hipMemcpyHostToDevice, stream)) !=
                hipSuccess)
                return cleanup({QMM_ERR_HIP, std::string("hipMemcpyAsync: ") + hipGetErrorString(e)});
        }
        if ((e = hipEventRecord(ev[b], stream)) != hipSuccess)
            return cleanup({QMM_ERR_HIP, std::string("hipEventRecord: ") + hipGetErrorString(e)});
    }
    return cleanup({QMM_OK, ""});
}

}  // namespace qmm
