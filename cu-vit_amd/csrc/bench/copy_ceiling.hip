// The HBM ceiling bench.py measures the memory-bound kernels against: a plain
// device copy of the same bytes, shaped to be the fastest copy found on gfx950
// (256-thread workgroups, eight per CU, each thread moving four 16-byte vectors
// per pass with non-temporal loads and stores, grid-stride over the buffer).
// Built into libcuvit_bench.so, apart from the product library: nothing but the
// benchmark calls it.
#include <hip/hip_runtime.h>

#include <cstdint>

namespace {

typedef unsigned int Vector __attribute__((ext_vector_type(4)));

constexpr int kThreads = 256;
constexpr int kVectorsPerThread = 4;
constexpr int kWorkgroupsPerCu = 8;

__global__ __launch_bounds__(kThreads) void copy_vectors(const Vector* __restrict__ source,
                                                         Vector* __restrict__ target,
                                                         std::int64_t count) {
    const std::int64_t pass = static_cast<std::int64_t>(gridDim.x) * kThreads * kVectorsPerThread;
    for (std::int64_t base = static_cast<std::int64_t>(blockIdx.x) * kThreads * kVectorsPerThread +
                             threadIdx.x;
         base < count; base += pass) {
        Vector v[kVectorsPerThread];
#pragma unroll
        for (int u = 0; u < kVectorsPerThread; ++u) {
            const std::int64_t i = base + static_cast<std::int64_t>(u) * kThreads;
            if (i < count) {
                v[u] = __builtin_nontemporal_load(source + i);
            }
        }
#pragma unroll
        for (int u = 0; u < kVectorsPerThread; ++u) {
            const std::int64_t i = base + static_cast<std::int64_t>(u) * kThreads;
            if (i < count) {
                __builtin_nontemporal_store(v[u], target + i);
            }
        }
    }
}

}  // namespace

/// Copies @p bytes from @p source to @p target on @p stream. Both pointers must
/// be 16-byte aligned and @p bytes a multiple of 16. Returns 0 on success, 1 on
/// an argument that breaks those rules, 2 when the launch fails.
extern "C" int cuvit_bench_copy(const void* source, void* target, std::int64_t bytes,
                                hipStream_t stream) {
    if (bytes == 0) {
        return 0;
    }
    if (source == nullptr || target == nullptr || bytes < 0 || bytes % 16 != 0 ||
        reinterpret_cast<std::uintptr_t>(source) % 16 != 0 ||
        reinterpret_cast<std::uintptr_t>(target) % 16 != 0) {
        return 1;
    }
    int device = 0;
    int cus = 0;
    if (hipGetDevice(&device) != hipSuccess ||
        hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device) != hipSuccess) {
        return 2;
    }
    const std::int64_t count = bytes / 16;
    const std::int64_t needed = (count + kThreads * kVectorsPerThread - 1) / (kThreads * kVectorsPerThread);
    const std::int64_t resident = static_cast<std::int64_t>(cus) * kWorkgroupsPerCu;
    const unsigned grid = static_cast<unsigned>(needed < resident ? needed : resident);
    copy_vectors<<<grid, kThreads, 0, stream>>>(static_cast<const Vector*>(source),
                                                static_cast<Vector*>(target), count);
    return hipGetLastError() == hipSuccess ? 0 : 2;
}
