// The disk tier's record reader (moelab/store.py:229-255, 378-445: ExpertStore.read with direct
// reads and split reads), host code only. A record is read as `parts` byte ranges in flight at
// once (an NVMe drive reaches its bandwidth only with several requests queued), each range
// aligned to 4096 bytes, on a pool of reader threads the library keeps for the life of the
// process. A range whose destination, file offset and length are all multiples of 4096 goes
// through the O_DIRECT descriptor (no copy through the page cache) when the caller passes one;
// a refused direct read (EINVAL: the file system does not support it; EFAULT: the buffer cannot
// be pinned for DMA) falls back to the ordinary descriptor and is counted.

#include <errno.h>
#include <string.h>
#include <unistd.h>

#include <condition_variable>
#include <deque>
#include <functional>
#include <memory>
#include <mutex>
#include <thread>
#include <vector>

#include "common.hpp"

namespace moehip {
namespace {

constexpr size_t kAlign = 4096;
constexpr int kMaxReaders = 16;

// one call's ranges: the calling thread waits until `left` is 0 (shared with the reader tasks, so
// the last one to finish may still release the lock after the caller has returned)
struct ReadJob {
    std::mutex mu;
    std::condition_variable cv;
    int left = 0;
    int direct_ranges = 0;
    int fallbacks = 0;
    int err = 0;          // first errno seen (0: none)
    long short_at = -1;   // offset of the first short read
    long got = 0, want = 0;
};

class ReaderPool {
  public:
    static ReaderPool &get() {
        static ReaderPool pool;
        return pool;
    }
    void submit(std::function<void()> f) {
        {
            std::lock_guard<std::mutex> l(mu_);
            q_.push_back(std::move(f));
        }
        cv_.notify_one();
    }

  private:
    ReaderPool() {
        unsigned n = std::thread::hardware_concurrency();
        n = n == 0 ? 4 : (n > kMaxReaders ? kMaxReaders : n);
        for (unsigned i = 0; i < n; ++i) threads_.emplace_back([this] { run(); });
    }
    ~ReaderPool() {
        {
            std::lock_guard<std::mutex> l(mu_);
            stop_ = true;
        }
        cv_.notify_all();
        for (auto &t : threads_) t.join();
    }
    void run() {
        for (;;) {
            std::function<void()> f;
            {
                std::unique_lock<std::mutex> l(mu_);
                cv_.wait(l, [this] { return stop_ || !q_.empty(); });
                if (q_.empty()) return;
                f = std::move(q_.front());
                q_.pop_front();
            }
            f();
        }
    }
    std::mutex mu_;
    std::condition_variable cv_;
    std::deque<std::function<void()>> q_;
    std::vector<std::thread> threads_;
    bool stop_ = false;
};

// pread until n bytes or end of file / error; returns bytes read, -errno on error
long pread_full(int fd, uint8_t *dst, size_t n, off_t off) {
    size_t done = 0;
    while (done < n) {
        const ssize_t r = pread(fd, dst + done, n - done, off + (off_t)done);
        if (r < 0) {
            if (errno == EINTR) continue;
            return -(long)errno;
        }
        if (r == 0) break;
        done += (size_t)r;
    }
    return (long)done;
}

void read_range(ReadJob *job, int fd, int fd_direct, uint8_t *dst, size_t n, off_t off) {
    bool direct = false, fell_back = false;
    long got = -1;
    const bool aligned = ((uintptr_t)dst % kAlign) == 0 && (off % (off_t)kAlign) == 0 && (n % kAlign) == 0;
    if (fd_direct >= 0 && aligned) {
        got = pread_full(fd_direct, dst, n, off);
        // EINVAL: no direct reads on this file system; EFAULT: memory the kernel cannot pin for
        // DMA (e.g. host memory mapped for the GPU): both fall back to the ordinary read
        if (got == -(long)EINVAL || got == -(long)EFAULT) {
            fell_back = true;
            got = -1;
        } else {
            direct = true;
        }
    }
    if (got == -1 && !direct) got = pread_full(fd, dst, n, off);
    std::lock_guard<std::mutex> l(job->mu);
    if (direct) ++job->direct_ranges;
    if (fell_back) ++job->fallbacks;
    if (got < 0) {
        if (job->err == 0) job->err = (int)-got;
    } else if ((size_t)got != n && job->short_at < 0) {
        job->short_at = (long)off;
        job->got = got;
        job->want = (long)n;
    }
    if (--job->left == 0) job->cv.notify_all();
}

}  // namespace
}  // namespace moehip

using namespace moehip;

extern "C" int moehip_disk_read(int fd, int fd_direct, int64_t offset, void *dst, size_t bytes, int parts,
                                int *direct_ranges, int *fallbacks) {
    MOEHIP_REQUIRE(fd >= 0 && dst != nullptr && offset >= 0 && bytes > 0, "disk_read: fd=%d dst=%p offset=%lld bytes=%zu",
                   fd, dst, (long long)offset, bytes);
    MOEHIP_REQUIRE(parts >= 1 && parts <= 64, "disk_read: parts=%d (1..64)", parts);
    // ranges of ceil(bytes / parts) rounded up to 4096 (the last one shorter)
    size_t chunk = (bytes + (size_t)parts - 1) / (size_t)parts;
    chunk = (chunk + kAlign - 1) / kAlign * kAlign;
    const int n = (int)((bytes + chunk - 1) / chunk);
    auto jp = std::make_shared<ReadJob>();
    ReadJob &job = *jp;
    job.left = n;
    uint8_t *d = static_cast<uint8_t *>(dst);
    if (n == 1) {
        read_range(&job, fd, fd_direct, d, bytes, (off_t)offset);
    } else {
        for (int i = 0; i < n; ++i) {
            const size_t o = (size_t)i * chunk;
            const size_t len = o + chunk <= bytes ? chunk : bytes - o;
            ReaderPool::get().submit([jp, fd, fd_direct, d, o, len, offset] {
                read_range(jp.get(), fd, fd_direct, d + o, len, (off_t)(offset + (int64_t)o));
            });
        }
        std::unique_lock<std::mutex> l(job.mu);
        job.cv.wait(l, [&job] { return job.left == 0; });
    }
    if (direct_ranges) *direct_ranges = job.direct_ranges;
    if (fallbacks) *fallbacks = job.fallbacks;
    if (job.err != 0) {
        set_error("disk_read: read failed at offset %lld (%zu bytes): %s", (long long)offset, bytes, strerror(job.err));
        return MOEHIP_EIO;
    }
    if (job.short_at >= 0) {
        set_error("disk_read: truncated read at offset %ld (%ld of %ld bytes)", job.short_at, job.got, job.want);
        return MOEHIP_EIO;
    }
    return MOEHIP_OK;
}
