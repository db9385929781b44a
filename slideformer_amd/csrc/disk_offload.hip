// slideformer_amd: asynchronous file offload of optimizer-state buffers (host code only).
//
// The reference offloads a fraction of the per-layer Adam moments to NVMe with
// tensornvme's DiskOffloader (layer_adam.py:92-106, 200-247): async_write /
// async_read of whole flat buffers, then sync_write_events / sync_read_events
// as fences around each layer's step.  This is the same contract on a pool of
// worker threads doing positioned reads and writes (pread/pwrite) in 64 MiB
// pieces, one file per buffer key under the offload directory, named
// "offload-<pid>-<key>" (the reference cleans "offload-*", layer_adam.py:122).

#include <fcntl.h>
#include <sys/stat.h>
#include <sys/types.h>
#include <unistd.h>

#include <cerrno>
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

struct Job {
    int fd;
    uint64_t off;
    char* ptr;
    uint64_t bytes;
    bool write;
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
};

namespace {

void worker_loop(la_disk* d)
{
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
        uint64_t done = 0;
        while (done < j.bytes) {
            const ssize_t r = j.write ? ::pwrite(j.fd, j.ptr + done, j.bytes - done, static_cast<off_t>(j.off + done))
                                      : ::pread(j.fd, j.ptr + done, j.bytes - done, static_cast<off_t>(j.off + done));
            if (r < 0) {
                if (errno == EINTR) continue;
                err = -errno;
                break;
            }
            if (r == 0) {  // short file on read
                err = -EIO;
                break;
            }
            done += static_cast<uint64_t>(r);
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
        fd = ::open(path.c_str(), O_RDWR | O_CREAT | O_TRUNC | O_CLOEXEC, 0600);
        if (fd < 0) return -errno;
        d->fds[key] = fd;
        d->paths.push_back(path);
    } else {
        fd = it->second;
    }
    char* p = static_cast<char*>(buf);
    for (uint64_t off = 0; off < bytes; off += kPiece) {
        const uint64_t k = bytes - off < kPiece ? bytes - off : kPiece;
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
    if (!out || !dir || !*dir) return LA_EINVAL;
    *out = nullptr;
    struct stat st;
    if (::stat(dir, &st) != 0) return -errno;
    if (!S_ISDIR(st.st_mode)) return -ENOTDIR;
    if (threads < 1) threads = 1;
    if (threads > 64) threads = 64;
    la_disk* d = new (std::nothrow) la_disk();
    if (!d) return -ENOMEM;
    d->dir = dir;
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
