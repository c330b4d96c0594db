// launch.hip -- grid sizing shared by every launcher.
#include <hip/hip_runtime.h>

#include <atomic>

#include "elementwise.hpp"
#include "spline_ops_hip.h"

namespace pt {

DeviceShape device_shape() {
    // One entry per device, filled on first use; the attribute never changes.
    static std::atomic<int> cached_cus[64];
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) dev = 0;
    int cus = cached_cus[dev].load(std::memory_order_relaxed);
    if (cus <= 0) {
        if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
            cus <= 0)
            cus = 256;
        cached_cus[dev].store(cus, std::memory_order_relaxed);
    }
    return DeviceShape{cus};
}

int64_t grid_one_pass(int64_t n_items) {
    const int64_t need = (n_items + kBlock - 1) / kBlock;
    // HSA grid sizes count work-items in 32 bits.
    const int64_t limit = 0xffffffffll / kBlock;
    return need < 1 ? 1 : (need > limit ? limit : need);
}

}  // namespace pt

extern "C" int spline_hip_grid_for(int64_t size, int streams, int64_t* grid_out, int* cus_out) {
    if (size < 0 || streams <= 0) return hipErrorInvalidValue;
    if (grid_out) *grid_out = pt::grid_one_pass(size >> 3);
    if (cus_out) *cus_out = pt::device_shape().cus;
    return hipSuccess;
}
