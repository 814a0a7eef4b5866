// hx_once.h — per-key memo of host-side queries (kernel attribute grants, device properties).
// The first caller for a key computes the value while holding the memo's lock, so every key is
// computed exactly once; every later caller reads the stored value. Safe from any number of host
// threads. Host code only (no HIP types), so host-only tests can exercise it.
#pragma once

#include <map>
#include <mutex>

namespace hx {

template <typename Key, typename Value>
class OnceMap {
public:
    template <typename F>
    Value get(const Key& k, F&& compute) {
        std::lock_guard<std::mutex> lock(mu_);
        auto it = m_.find(k);
        if (it != m_.end()) return it->second;
        const Value v = compute();
        m_.emplace(k, v);
        return v;
    }
    size_t size() const {
        std::lock_guard<std::mutex> lock(mu_);
        return m_.size();
    }

private:
    mutable std::mutex mu_;
    std::map<Key, Value> m_;
};

}  // namespace hx
