// Host-only driver for the native file offloader (la_disk_*), built with g++
// under AddressSanitizer/UndefinedBehaviorSanitizer or ThreadSanitizer by
// tests/test_native_sanitizers.py.  Exercises concurrent writers/readers on
// the worker pool, multi-piece transfers, error paths and teardown, with
// buffered and with direct (O_DIRECT) I/O.
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <thread>
#include <vector>

#include "layer_adam.h"

#define CHECK(c)                                                   \
    do {                                                           \
        if (!(c)) {                                                \
            std::fprintf(stderr, "check failed: %s (line %d)\n", #c, __LINE__); \
            return 1;                                              \
        }                                                          \
    } while (0)

// The whole sequence in one mode (flags 0: buffered; LA_DISK_DIRECT: O_DIRECT).
static int run(const char* dir, unsigned flags)
{
    la_disk_t* d = nullptr;
    CHECK(la_disk_create_ex(dir, 8, flags, &d) == 0 && d);
    CHECK(la_disk_destroy(d) == 0);
    CHECK(la_disk_create_ex("/nonexistent/dir/x", 2, flags, &d) != 0);
    CHECK(la_disk_create_ex(dir, 2, 0x80u, &d) != 0);  // unknown flag
    CHECK(la_disk_create_ex(dir, 8, flags, &d) == 0);

    // buffers of several sizes, one spanning two 64 MiB pieces (five 16 MiB
    // pieces in direct mode, whose last one is not a whole block)
    const std::vector<uint64_t> sizes = {1, 4096, 1000003, (65ull << 20) + 12345};
    std::vector<std::vector<unsigned char>> src(sizes.size()), dst(sizes.size());
    for (size_t i = 0; i < sizes.size(); ++i) {
        src[i].resize(sizes[i]);
        dst[i].assign(sizes[i], 0);
        for (uint64_t k = 0; k < sizes[i]; ++k) src[i][k] = static_cast<unsigned char>((k * 131 + i * 7 + flags) & 0xff);
    }
    CHECK(la_disk_read_async(d, 999, dst[0].data(), 1) < 0);  // never written: -ENOENT
    // writes submitted from several threads at once
    std::vector<std::thread> ts;
    for (size_t i = 0; i < sizes.size(); ++i)
        ts.emplace_back([&, i] { la_disk_write_async(d, 100 + i, src[i].data(), sizes[i]); });
    for (auto& t : ts) t.join();
    CHECK(la_disk_sync_writes(d) == 0);
    ts.clear();
    for (size_t i = 0; i < sizes.size(); ++i)
        ts.emplace_back([&, i] { la_disk_read_async(d, 100 + i, dst[i].data(), sizes[i]); });
    for (auto& t : ts) t.join();
    CHECK(la_disk_sync_reads(d) == 0);
    for (size_t i = 0; i < sizes.size(); ++i) CHECK(std::memcmp(src[i].data(), dst[i].data(), sizes[i]) == 0);
    // a read longer than the file fails with an error, not a crash
    std::vector<unsigned char> big(8192);
    CHECK(la_disk_read_async(d, 100, big.data(), big.size()) == 0);
    CHECK(la_disk_sync_reads(d) < 0);
    // overwrite and re-read
    for (auto& b : src[2]) b ^= 0x5a;
    CHECK(la_disk_write_async(d, 102, src[2].data(), sizes[2]) == 0);
    CHECK(la_disk_sync_writes(d) == 0);
    CHECK(la_disk_read_async(d, 102, dst[2].data(), sizes[2]) == 0);
    CHECK(la_disk_sync_reads(d) == 0);
    CHECK(std::memcmp(src[2].data(), dst[2].data(), sizes[2]) == 0);
    // a block-aligned buffer of whole blocks (straight to the file in direct
    // mode) and the same bytes read back into an unaligned one
    const uint64_t an = (33ull << 20) + 8192;
    unsigned char* al = static_cast<unsigned char*>(std::aligned_alloc(4096, an));
    CHECK(al != nullptr);
    for (uint64_t k = 0; k < an; ++k) al[k] = static_cast<unsigned char>((k * 7 + 3) & 0xff);
    std::vector<unsigned char> back(an + 1, 0);
    CHECK(la_disk_write_async(d, 300, al, an) == 0);
    CHECK(la_disk_sync_writes(d) == 0);
    CHECK(la_disk_read_async(d, 300, back.data() + 1, an) == 0);
    CHECK(la_disk_sync_reads(d) == 0);
    CHECK(std::memcmp(al, back.data() + 1, an) == 0);
    std::free(al);
    // teardown with work still queued
    CHECK(la_disk_write_async(d, 200, src[3].data(), sizes[3]) == 0);
    CHECK(la_disk_destroy(d) == 0);
    CHECK(la_disk_destroy(nullptr) == 0);
    return 0;
}

int main(int argc, char** argv)
{
    if (argc < 2) return 2;
    la_disk_t* d = nullptr;
    CHECK(la_disk_create(argv[1], 8, &d) == 0 && d);  // the flag-less entry point
    CHECK(la_disk_destroy(d) == 0);
    if (run(argv[1], 0u) != 0) return 1;
    if (run(argv[1], LA_DISK_DIRECT) != 0) return 1;
    std::printf("disk offload driver ok\n");
    return 0;
}
