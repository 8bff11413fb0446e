// pj_host_lock.h — host-side locks of per-device library state.
#pragma once
#include <mutex>

namespace pj {

constexpr int PJ_LOCK_DEVICES = 64;

// The lock of `device`'s fixed no-allocation encode scratch (one array per
// GPU, shared by every context on it).  pj_encode_device_noalloc holds it
// from the kernel that clears the scratch until its stream has drained, so
// calls on one GPU from different threads or contexts run one after the
// other instead of clearing each other's look-back words mid-kernel.
// Taking a std::mutex allocates nothing.
inline std::mutex &noalloc_lock(int device) {
    static std::mutex m[PJ_LOCK_DEVICES];
    return m[device < 0 || device >= PJ_LOCK_DEVICES ? 0 : device];
}

}  // namespace pj
