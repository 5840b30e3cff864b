// CPU check of OncePerDevice (acestep.cpp_amd/csrc/once_per_device.h), the
// guard behind the per-device hipFuncSetAttribute of the decode kernel:
// 8 threads x 200 calls over devices 0..3 set each device exactly once; a
// failing setting is retried on the next call; a new device id is set on
// first use.  Prints "key value" lines.
#include <atomic>
#include <cstdio>
#include <thread>
#include <vector>

#include "once_per_device.h"

int main() {
    mxfa::OncePerDevice g;
    std::atomic<int> calls[8];
    for (auto &c : calls) c = 0;
    std::vector<std::thread> ts;
    for (int t = 0; t < 8; t++)
        ts.emplace_back([&, t] {
            for (int i = 0; i < 200; i++) {
                const int dev = (t + i) % 4;
                const int r = g.run(dev, [&] { calls[dev]++; return 0; });
                if (r != 0) std::printf("bad_return %d\n", r);
            }
        });
    for (auto &t : ts) t.join();
    std::printf("dev0 %d\ndev1 %d\ndev2 %d\ndev3 %d\n", calls[0].load(), calls[1].load(), calls[2].load(),
                calls[3].load());
    // a failure is not remembered: the next call retries
    int tries = 0;
    const int r1 = g.run(5, [&] { tries++; return 7; });
    const int r2 = g.run(5, [&] { tries++; return 0; });
    const int r3 = g.run(5, [&] { tries++; return 0; });
    std::printf("retry %d %d %d %d\n", r1, r2, r3, tries);
    // device 7 after 5: the table grows, the others keep their state
    const int r4 = g.run(7, [&] { calls[7]++; return 0; });
    const int r5 = g.run(0, [&] { calls[0]++; return 0; });
    std::printf("grow %d %d %d %d\n", r4, r5, calls[7].load(), calls[0].load());
    return 0;
}
