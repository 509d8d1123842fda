// Grid shaping shared by the launch functions.
#include "launch.hpp"

#include <atomic>

namespace cuvit::detail {
namespace {

constexpr int kMaxDevices = 64;
/// Compute units of a gfx950 MI355X, used if the attribute query fails.
constexpr int kDefaultComputeUnits = 256;

std::atomic<int> cached_units[kMaxDevices];

} // namespace

int compute_units() {
    int device = 0;
    if (hipGetDevice(&device) != hipSuccess || device < 0 || device >= kMaxDevices) {
        return kDefaultComputeUnits;
    }
    int units = cached_units[device].load(std::memory_order_relaxed);
    if (units > 0) {
        return units;
    }
    if (hipDeviceGetAttribute(&units, hipDeviceAttributeMultiprocessorCount, device) !=
            hipSuccess ||
        units <= 0) {
        units = kDefaultComputeUnits;
    }
    cached_units[device].store(units, std::memory_order_relaxed);
    return units;
}

hipError_t allow_lds(const void* kernel, std::size_t bytes, std::atomic<std::uint64_t>& devices) {
    if (bytes <= 65536) {
        return hipSuccess;
    }
    int device = 0;
    if (hipGetDevice(&device) != hipSuccess || device < 0 || device >= 64) {
        return hipFuncSetAttribute(kernel, hipFuncAttributeMaxDynamicSharedMemorySize,
                                   static_cast<int>(bytes));
    }
    const std::uint64_t bit = std::uint64_t{1} << device;
    if ((devices.load(std::memory_order_acquire) & bit) != 0) {
        return hipSuccess;
    }
    const hipError_t result =
        hipFuncSetAttribute(kernel, hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(bytes));
    if (result == hipSuccess) {
        devices.fetch_or(bit, std::memory_order_acq_rel);
    }
    return result;
}

unsigned int stride_grid(std::int64_t units, int units_per_block, int cap_per_cu) {
    const std::int64_t needed = (units + units_per_block - 1) / units_per_block;
    const std::int64_t cap = static_cast<std::int64_t>(compute_units()) * cap_per_cu;
    const std::int64_t blocks = needed < cap ? needed : cap;
    return static_cast<unsigned int>(blocks > 0 ? blocks : 1);
}

} // namespace cuvit::detail
