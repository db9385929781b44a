// slideformer_amd: asynchronous file offload of optimizer-state buffers (host code only).
//
// The reference offloads a fraction of the per-layer Adam moments to NVMe with
// tensornvme's DiskOffloader (layer_adam.py:92-106, 200-247): async_write /
// async_read of whole flat buffers, then sync_write_events / sync_read_events
// as fences around each layer's step.  This is the same contract on a pool of
// worker threads doing positioned reads and writes (pread/pwrite) in 64 MiB
// pieces, one file per buffer key under the offload directory, named
// "offload-<pid>-<key>" (the reference cleans "offload-*", layer_adam.py:122).
//
// Direct mode (LA_DISK_DIRECT) opens the files with O_DIRECT, so the moments
// moved out of host RAM do not stay there as cached pages and the rates are
// the device's.  O_DIRECT needs the buffer address, the file offset and the
// length to be multiples of the device block; pieces are 16 MiB at offsets
// that are multiples of 16 MiB, a piece whose buffer is aligned goes straight
// to the device, any other is copied through an aligned bounce buffer of its
// worker, and the last piece of a buffer is padded with zeros to a whole
// block (the file is that much longer; a read copies out only the bytes
// asked for).

#include <fcntl.h>
#include <sys/stat.h>
#include <sys/types.h>
#include <unistd.h>

#include <cerrno>
#include <cstdlib>
#include <cstring>
#include <memory>
#include <condition_variable>
#include <cstdint>
#include <cstdio>
#include <deque>
#include <mutex>
#include <new>
#include <string>
#include <thread>
#include <unordered_map>
#include <vector>

#include "../../include/layer_adam.h"

namespace {

constexpr uint64_t kPiece = 64ull << 20;
constexpr uint64_t kDirectPiece = 16ull << 20;  // direct mode: also each worker's bounce buffer
constexpr uint64_t kBlock = 4096;                // O_DIRECT alignment (covers 512 B and 4 KiB devices)

struct Job {
    int fd;
    uint64_t off;
    char* ptr;
    uint64_t bytes;
    bool write;
};

uint64_t round_up(uint64_t x, uint64_t a) { return (x + a - 1) / a * a; }

struct FreeDeleter {
    void operator()(char* p) const { std::free(p); }
};

}  // namespace

struct la_disk {
    std::string dir;
    std::vector<std::thread> workers;
    std::mutex mu;
    std::condition_variable work_cv, done_cv;
    std::deque<Job> queue;
    bool stop = false;
    uint64_t pending_w = 0, pending_r = 0;
    int err_w = 0, err_r = 0;
    std::unordered_map<uint64_t, int> fds;
    std::vector<std::string> paths;
    bool direct = false;
};

namespace {

// All `bytes` at `ptr` to or from the file at `off`; 0 or a negative errno.
int transfer(int fd, char* ptr, uint64_t bytes, uint64_t off, bool write)
{
    uint64_t done = 0;
    while (done < bytes) {
        const ssize_t r = write ? ::pwrite(fd, ptr + done, bytes - done, static_cast<off_t>(off + done))
                                : ::pread(fd, ptr + done, bytes - done, static_cast<off_t>(off + done));
        if (r < 0) {
            if (errno == EINTR) continue;
            return -errno;
        }
        if (r == 0) return -EIO;  // short file on read
        done += static_cast<uint64_t>(r);
    }
    return 0;
}

void worker_loop(la_disk* d)
{
    std::unique_ptr<char, FreeDeleter> bounce;  // direct mode, allocated on first need
    for (;;) {
        Job j;
        {
            std::unique_lock<std::mutex> lk(d->mu);
            d->work_cv.wait(lk, [d] { return d->stop || !d->queue.empty(); });
            if (d->queue.empty()) return;  // stop requested and nothing left
            j = d->queue.front();
            d->queue.pop_front();
        }
        int err = 0;
        const bool aligned = reinterpret_cast<uintptr_t>(j.ptr) % kBlock == 0 && j.bytes % kBlock == 0;
        if (!d->direct || aligned) {
            err = transfer(j.fd, j.ptr, j.bytes, j.off, j.write);
        } else {
            if (!bounce) bounce.reset(static_cast<char*>(std::aligned_alloc(kBlock, kDirectPiece)));
            if (!bounce) {
                err = -ENOMEM;
            } else {
                const uint64_t padded = round_up(j.bytes, kBlock);
                if (j.write) {
                    std::memcpy(bounce.get(), j.ptr, j.bytes);
                    std::memset(bounce.get() + j.bytes, 0, padded - j.bytes);
                    err = transfer(j.fd, bounce.get(), padded, j.off, true);
                } else {
                    err = transfer(j.fd, bounce.get(), padded, j.off, false);
                    if (!err) std::memcpy(j.ptr, bounce.get(), j.bytes);
                }
            }
        }
        {
            std::lock_guard<std::mutex> lk(d->mu);
            if (j.write) {
                if (err && !d->err_w) d->err_w = err;
                --d->pending_w;
            } else {
                if (err && !d->err_r) d->err_r = err;
                --d->pending_r;
            }
        }
        d->done_cv.notify_all();
    }
}

int submit(la_disk* d, uint64_t key, void* buf, uint64_t bytes, bool write)
try {
    if (!d || (bytes > 0 && !buf)) return LA_EINVAL;
    std::lock_guard<std::mutex> lk(d->mu);
    auto it = d->fds.find(key);
    int fd;
    if (it == d->fds.end()) {
        if (!write) return -ENOENT;  // nothing was ever written under this key
        char name[96];
        std::snprintf(name, sizeof(name), "/offload-%d-%llu", static_cast<int>(::getpid()),
                      static_cast<unsigned long long>(key));
        const std::string path = d->dir + name;
        fd = ::open(path.c_str(), O_RDWR | O_CREAT | O_TRUNC | O_CLOEXEC | (d->direct ? O_DIRECT : 0), 0600);
        if (fd < 0) return -errno;
        d->fds[key] = fd;
        d->paths.push_back(path);
    } else {
        fd = it->second;
    }
    char* p = static_cast<char*>(buf);
    const uint64_t piece = d->direct ? kDirectPiece : kPiece;
    for (uint64_t off = 0; off < bytes; off += piece) {
        const uint64_t k = bytes - off < piece ? bytes - off : piece;
        d->queue.push_back(Job{fd, off, p + off, k, write});
        if (write) ++d->pending_w;
        else ++d->pending_r;
    }
    d->work_cv.notify_all();
    return LA_OK;
} catch (...) {
    return -ENOMEM;
}

}  // namespace

extern "C" {

int la_disk_create(const char* dir, int threads, la_disk_t** out)
{
    return la_disk_create_ex(dir, threads, 0u, out);
}

int la_disk_create_ex(const char* dir, int threads, unsigned flags, la_disk_t** out)
{
    if (!out || !dir || !*dir || (flags & ~LA_DISK_DIRECT)) return LA_EINVAL;
    *out = nullptr;
    struct stat st;
    if (::stat(dir, &st) != 0) return -errno;
    if (!S_ISDIR(st.st_mode)) return -ENOTDIR;
    if (flags & LA_DISK_DIRECT) {
        // the file system must take O_DIRECT; find out now rather than at the first write
        char name[96];
        std::snprintf(name, sizeof(name), "/offload-%d-direct-probe", static_cast<int>(::getpid()));
        const std::string probe = std::string(dir) + name;
        const int fd = ::open(probe.c_str(), O_RDWR | O_CREAT | O_TRUNC | O_CLOEXEC | O_DIRECT, 0600);
        if (fd < 0) return -errno;
        ::close(fd);
        ::unlink(probe.c_str());
    }
    if (threads < 1) threads = 1;
    if (threads > 64) threads = 64;
    la_disk* d = new (std::nothrow) la_disk();
    if (!d) return -ENOMEM;
    d->dir = dir;
    d->direct = (flags & LA_DISK_DIRECT) != 0;
    try {
        for (int i = 0; i < threads; ++i) d->workers.emplace_back(worker_loop, d);
    } catch (...) {
        // no exception crosses the C ABI: stop the workers already started
        {
            std::lock_guard<std::mutex> lk(d->mu);
            d->stop = true;
        }
        d->work_cv.notify_all();
        for (auto& t : d->workers) t.join();
        delete d;
        return -EAGAIN;
    }
    *out = d;
    return LA_OK;
}

int la_disk_write_async(la_disk_t* d, uint64_t key, const void* src, uint64_t bytes)
{
    return submit(d, key, const_cast<void*>(src), bytes, true);
}

int la_disk_read_async(la_disk_t* d, uint64_t key, void* dst, uint64_t bytes)
{
    return submit(d, key, dst, bytes, false);
}

int la_disk_sync_writes(la_disk_t* d)
{
    if (!d) return LA_EINVAL;
    std::unique_lock<std::mutex> lk(d->mu);
    d->done_cv.wait(lk, [d] { return d->pending_w == 0; });
    const int e = d->err_w;
    d->err_w = 0;
    return e;
}

int la_disk_sync_reads(la_disk_t* d)
{
    if (!d) return LA_EINVAL;
    std::unique_lock<std::mutex> lk(d->mu);
    d->done_cv.wait(lk, [d] { return d->pending_r == 0; });
    const int e = d->err_r;
    d->err_r = 0;
    return e;
}

int la_disk_destroy(la_disk_t* d)
{
    if (!d) return LA_OK;
    {
        std::lock_guard<std::mutex> lk(d->mu);
        d->stop = true;
    }
    d->work_cv.notify_all();
    for (auto& t : d->workers) t.join();
    for (auto& kv : d->fds) ::close(kv.second);
    for (auto& p : d->paths) ::unlink(p.c_str());
    delete d;
    return LA_OK;
}

}  // extern "C"
