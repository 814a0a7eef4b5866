// once_threads.cpp — hammers hx::OnceMap (helixml_amd/csrc/hx_once.h) from many threads: every key
// must be computed exactly once and every reader must see the computed value. Built with
// -fsanitize=thread by tests/test_once_threads.py, which fails on any reported data race.
#include <atomic>
#include <cstdio>
#include <thread>
#include <tuple>
#include <vector>

#include "hx_once.h"

int main() {
    hx::OnceMap<std::tuple<const void*, int, size_t>, bool> grants;
    hx::OnceMap<int, int> cus;
    std::atomic<int> computed{0};
    std::atomic<int> wrong{0};
    static int kernels[8];
    std::vector<std::thread> ts;
    for (int t = 0; t < 8; ++t)
        ts.emplace_back([&, t] {
            for (int i = 0; i < 20000; ++i) {
                const int k = (i * 7 + t) % 8, dev = (i / 8) % 4;
                const size_t bytes = 1024u * (size_t)(k + 1);
                const bool g = grants.get(std::make_tuple((const void*)&kernels[k], dev, bytes), [&] {
                    computed.fetch_add(1);
                    return (k + dev) % 3 != 0;
                });
                if (g != ((k + dev) % 3 != 0)) wrong.fetch_add(1);
                const int c = cus.get(dev, [&] {
                    computed.fetch_add(1);
                    return 256 + dev;
                });
                if (c != 256 + dev) wrong.fetch_add(1);
            }
        });
    for (auto& th : ts) th.join();
    std::printf("computed %d (want %d), wrong %d, keys %zu + %zu\n", computed.load(), 8 * 4 + 4, wrong.load(),
                grants.size(), cus.size());
    return (computed.load() == 36 && wrong.load() == 0 && grants.size() == 32 && cus.size() == 4) ? 0 : 1;
}
