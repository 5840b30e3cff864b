// once_per_device.h -- a per-device, thread-safe "do this once" guard.
//
// Some HIP settings are per (function, device), for instance
// hipFuncSetAttribute(MaxDynamicSharedMemorySize) for a kernel that takes
// more than 64 KB of dynamic LDS: it applies to the current device only.
// The engine's entry points may be called from several host threads and on
// several devices, so such a setting is made once per device that launches
// the kernel, under a lock.  Host-only code (no HIP types): the CPU tests
// compile it on its own.
#pragma once

#include <mutex>
#include <vector>

namespace mxfa {

class OncePerDevice {
public:
    // Calls fn() the first time device `dev` is seen, and again on a later
    // call if fn() did not return 0 (a failed setting is retried); returns
    // fn()'s result, or 0 when the device is already done.  fn runs under
    // the guard's lock: concurrent callers for one device wait for it.
    template <typename F>
    auto run(int dev, F fn) -> decltype(fn()) {
        using R = decltype(fn());
        if (dev < 0) return fn();   // (a device id is never negative; nothing is cached)
        std::lock_guard<std::mutex> lock(mu_);
        if ((size_t)dev >= done_.size()) done_.resize((size_t)dev + 1, 0);
        if (done_[(size_t)dev]) return R(0);
        const R r = fn();
        if (r == R(0)) done_[(size_t)dev] = 1;
        return r;
    }

private:
    std::mutex mu_;
    std::vector<char> done_;
};

}  // namespace mxfa
