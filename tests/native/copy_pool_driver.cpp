// Drives la_host::CopyPool (slideformer_amd/csrc/copy_pool.h) the way the
// streaming pipeline does: many fork-join rounds of piece lists of varying
// length, back to back, with pools of several sizes created and destroyed.
// Every byte is checked.  Built with g++ under sanitizers by
// tests/test_native_sanitizers.py.
#include <algorithm>
#include <cstdio>
#include <cstdlib>
#include <vector>

#include "copy_pool.h"

using la_host::CopyPool;
using la_host::Piece;

static int check_round(CopyPool& pool, std::vector<char>& src, std::vector<char>& dst, uint64_t piece, int round)
{
    for (size_t i = 0; i < src.size(); ++i) src[i] = static_cast<char>((i * 131 + round * 7) & 0xff);
    std::vector<Piece> pieces;
    for (uint64_t o = 0; o < src.size(); o += piece) {
        const uint64_t b = (src.size() - o) < piece ? (src.size() - o) : piece;
        pieces.push_back(Piece{dst.data() + o, src.data() + o, b});
    }
    pool.run(pieces);
    for (size_t i = 0; i < src.size(); ++i)
        if (dst[i] != src[i]) {
            std::printf("mismatch at %zu in round %d\n", i, round);
            return 1;
        }
    return 0;
}

int main()
{
    for (int threads : {1, 2, 5, 8}) {
        CopyPool pool(threads);
        if (pool.threads() != threads) return 2;
        std::vector<Piece> none;
        pool.run(none);  // an empty round returns at once
        for (int round = 0; round < 200; ++round) {
            const size_t bytes = 1 + static_cast<size_t>(round) * 997 % 50000;
            std::vector<char> src(bytes), dst(bytes, 0);
            const uint64_t piece = 1 + round % 4096;
            if (check_round(pool, src, dst, piece, round)) return 1;
        }
    }
    // copies through the nontemporal path: every destination/source phase,
    // sizes just below and above its thresholds
    {
        CopyPool pool(4);
        std::vector<char> src(1 << 16), dst(1 << 16);
        for (size_t i = 0; i < src.size(); ++i) src[i] = static_cast<char>(i * 7 + 3);
        for (int doff = 0; doff < 16; ++doff)
            for (int soff = 0; soff < 16; soff += 5)
                for (uint64_t bytes : {1ull, 255ull, 256ull, 271ull, 272ull, 300ull, 4096ull + 17, 40000ull}) {
                    std::fill(dst.begin(), dst.end(), 0);
                    std::vector<Piece> one{Piece{dst.data() + doff, src.data() + soff, bytes}};
                    pool.run(one);
                    for (uint64_t k = 0; k < bytes; ++k)
                        if (dst[doff + k] != src[soff + k]) {
                            std::printf("nt copy mismatch doff %d soff %d bytes %llu at %llu\n", doff, soff,
                                        static_cast<unsigned long long>(bytes), static_cast<unsigned long long>(k));
                            return 1;
                        }
                    if (dst[doff + bytes] != 0 || (doff > 0 && dst[doff - 1] != 0)) {
                        std::printf("nt copy wrote outside its range\n");
                        return 1;
                    }
                }
    }
    // pools that are destroyed without ever running, and right after a run
    for (int i = 0; i < 20; ++i) {
        CopyPool idle(4);
        CopyPool used(3);
        std::vector<char> src(12345), dst(12345);
        if (check_round(used, src, dst, 1000, i)) return 1;
    }
    std::printf("copy pool driver ok\n");
    return 0;
}
