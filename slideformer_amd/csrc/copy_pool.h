// Fork-join pool of host threads that copies a list of memory pieces.  Used
// by the streaming pipeline for the copies between pageable host arrays and
// page-locked staging.  Plain C++17, no HIP.
#ifndef SLIDEFORMER_AMD_COPY_POOL_H
#define SLIDEFORMER_AMD_COPY_POOL_H

#include <atomic>
#include <condition_variable>
#include <cstdint>
#include <cstring>
#include <mutex>
#include <thread>
#include <vector>
#if defined(__x86_64__)
#include <emmintrin.h>
#endif

namespace la_host {

// Copy `bytes` from src to dst.  The bulk goes through 16-byte nontemporal
// stores (SSE2, part of every x86-64): the destination is written once and
// not read back by this thread, so it should neither be read for ownership
// nor evict the source from the caches.  Unaligned edges use memcpy.  Returns
// true when nontemporal stores were issued (the caller then fences).
#ifndef LA_COPY_NT
#define LA_COPY_NT 1
#endif

inline bool copy_streaming(char* dst, const char* src, uint64_t bytes)
{
#if defined(__x86_64__) && LA_COPY_NT
    const uint64_t head = (16u - (reinterpret_cast<uintptr_t>(dst) & 15u)) & 15u;
    if (bytes < head + 256) {
        std::memcpy(dst, src, bytes);
        return false;
    }
    std::memcpy(dst, src, head);
    dst += head;
    src += head;
    bytes -= head;
    const uint64_t body = bytes & ~static_cast<uint64_t>(63);
    for (uint64_t o = 0; o < body; o += 64) {
        const __m128i a = _mm_loadu_si128(reinterpret_cast<const __m128i*>(src + o));
        const __m128i b = _mm_loadu_si128(reinterpret_cast<const __m128i*>(src + o + 16));
        const __m128i c = _mm_loadu_si128(reinterpret_cast<const __m128i*>(src + o + 32));
        const __m128i d = _mm_loadu_si128(reinterpret_cast<const __m128i*>(src + o + 48));
        _mm_stream_si128(reinterpret_cast<__m128i*>(dst + o), a);
        _mm_stream_si128(reinterpret_cast<__m128i*>(dst + o + 16), b);
        _mm_stream_si128(reinterpret_cast<__m128i*>(dst + o + 32), c);
        _mm_stream_si128(reinterpret_cast<__m128i*>(dst + o + 48), d);
    }
    std::memcpy(dst + body, src + body, bytes - body);
    return true;
#else
    std::memcpy(dst, src, bytes);
    return false;
#endif
}

struct Piece {
    char* dst;
    const char* src;
    uint64_t bytes;
};

// run() hands a list of pieces to the workers and the calling thread and
// returns when every piece is copied.  One run() at a time per pool.
class CopyPool {
public:
    // `threads` counts the calling thread: threads - 1 workers are started.
    // Throws std::system_error if a thread cannot be started (none is left running).
    explicit CopyPool(int threads)
    {
        try {
            for (int i = 1; i < threads; ++i) workers_.emplace_back([this] { loop(); });
        } catch (...) {
            shutdown();
            throw;
        }
    }
    ~CopyPool() { shutdown(); }
    CopyPool(const CopyPool&) = delete;
    CopyPool& operator=(const CopyPool&) = delete;
    int threads() const { return static_cast<int>(workers_.size()) + 1; }

    void run(const std::vector<Piece>& pieces)
    {
        if (pieces.empty()) return;
        {
            std::lock_guard<std::mutex> g(mu_);
            job_ = &pieces;
            next_.store(0);
            busy_ = workers_.size();
            ++gen_;
        }
        cv_work_.notify_all();
        drain(pieces);
        std::unique_lock<std::mutex> lk(mu_);
        cv_done_.wait(lk, [this] { return busy_ == 0; });
        job_ = nullptr;
    }

private:
    void shutdown()
    {
        {
            std::lock_guard<std::mutex> g(mu_);
            stop_ = true;
        }
        cv_work_.notify_all();
        for (std::thread& t : workers_)
            if (t.joinable()) t.join();
        workers_.clear();
    }
    void drain(const std::vector<Piece>& pieces)
    {
        bool streamed = false;
        for (;;) {
            const size_t i = next_.fetch_add(1);
            if (i >= pieces.size()) break;
            streamed |= copy_streaming(pieces[i].dst, pieces[i].src, pieces[i].bytes);
        }
#if defined(__x86_64__)
        // nontemporal stores are weakly ordered: make them globally visible
        // before run() reports the copy done (the copy engines read them next)
        if (streamed) _mm_sfence();
#endif
    }
    void loop()
    {
        uint64_t seen = 0;
        std::unique_lock<std::mutex> lk(mu_);
        for (;;) {
            cv_work_.wait(lk, [&] { return stop_ || gen_ != seen; });
            if (stop_) return;
            seen = gen_;
            const std::vector<Piece>* job = job_;
            lk.unlock();
            drain(*job);
            lk.lock();
            if (--busy_ == 0) cv_done_.notify_one();
        }
    }

    std::vector<std::thread> workers_;
    std::mutex mu_;
    std::condition_variable cv_work_, cv_done_;
    const std::vector<Piece>* job_ = nullptr;
    std::atomic<size_t> next_{0};
    size_t busy_ = 0;
    uint64_t gen_ = 0;
    bool stop_ = false;
};


}  // namespace la_host

#endif  // SLIDEFORMER_AMD_COPY_POOL_H
