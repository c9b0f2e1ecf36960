// q8_noalloc_owner.h -- who may use a device's no-allocation scratch.
//
// q8_matmul_noalloc quantizes its activations into one static device array
// per GPU (q8_noalloc.hip).  Two contexts on one GPU each run on a stream of
// their own, so their calls could overlap on that array.  The rule enforced
// here: the first context that uses a device's array holds it until it
// releases it (q8_close); while it is held, any other context is refused.
// Host-only, header-only (no HIP), so the CPU tests compile it on its own.
#ifndef Q8_NOALLOC_OWNER_H
#define Q8_NOALLOC_OWNER_H

#include <mutex>

namespace q8i {

class NoallocOwners {
public:
    static constexpr int kMaxDevices = 64;

    // True if `owner` holds `device`'s array after the call: it already held
    // it, or it was free and `owner` takes it.  False for another holder or a
    // device outside 0..kMaxDevices-1.
    bool claim(int device, const void *owner) {
        if (device < 0 || device >= kMaxDevices || !owner) return false;
        std::lock_guard<std::mutex> lock(mu_);
        if (!holder_[device]) holder_[device] = owner;
        return holder_[device] == owner;
    }

    // Frees every device `owner` holds.
    void release(const void *owner) {
        std::lock_guard<std::mutex> lock(mu_);
        for (const void *&h : holder_)
            if (h == owner) h = nullptr;
    }

    const void *holder(int device) {
        if (device < 0 || device >= kMaxDevices) return nullptr;
        std::lock_guard<std::mutex> lock(mu_);
        return holder_[device];
    }

private:
    std::mutex mu_;
    const void *holder_[kMaxDevices] = {};
};

}  // namespace q8i

#endif
