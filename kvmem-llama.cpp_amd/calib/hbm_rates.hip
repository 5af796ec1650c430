// The HBM rates a plain streaming kernel reaches on this device: read only,
// write only and copy, 1 GiB each way, 16-byte accesses.  The byte-bound
// kernels of the library are judged against these as well as against the
// 8 TB/s headline.  Each workgroup of the read and copy kernels takes one
// contiguous 16 KiB piece (four nontemporal 16-byte loads per thread, all
// in flight) and exits; the write kernel stores one 16-byte word per thread
// with plain stores.  These measured fastest of 1-16 accesses per thread,
// 256-1024 threads, nontemporal or not, and grid-stride forms.  Prints one
// JSON line; medians of 15 timed launches (hipEvents on the launch stream)
// after 3 untimed ones.
//
//     hbm_rates [MiB]        (default 1024; a multiple of 16)
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdio>
#include <cstdlib>
#include <vector>

typedef unsigned int v4u __attribute__((ext_vector_type(4)));

#define CHECK(x)                                                                          \
    do {                                                                                  \
        hipError_t e_ = (x);                                                              \
        if (e_ != hipSuccess) {                                                           \
            std::fprintf(stderr, "hbm_rates: %s at line %d\n", hipGetErrorString(e_), __LINE__); \
            std::exit(1);                                                                 \
        }                                                                                 \
    } while (0)

constexpr int kThreads = 256;
constexpr int kLoads = 4;  // 16 KiB per workgroup

__global__ __launch_bounds__(kThreads) void read_kernel(const v4u *__restrict__ src, unsigned *__restrict__ sink) {
    const size_t base = static_cast<size_t>(blockIdx.x) * kThreads * kLoads + threadIdx.x;
    unsigned acc = 0;
#pragma unroll
    for (int i = 0; i < kLoads; ++i) {
        const v4u v = __builtin_nontemporal_load(src + base + static_cast<size_t>(i) * kThreads);
        acc ^= v.x ^ v.y ^ v.z ^ v.w;
    }
    if (acc == 0x9e3779b9u) {  // never: the source is filled with one byte value
        sink[0] = acc;
    }
}

__global__ __launch_bounds__(kThreads) void write_kernel(v4u *__restrict__ dst) {
    const v4u v = {1u, 2u, 3u, static_cast<unsigned>(threadIdx.x)};
    dst[static_cast<size_t>(blockIdx.x) * kThreads + threadIdx.x] = v;
}

__global__ __launch_bounds__(kThreads) void copy_kernel(const v4u *__restrict__ src, v4u *__restrict__ dst) {
    const size_t base = static_cast<size_t>(blockIdx.x) * kThreads * kLoads + threadIdx.x;
    v4u v[kLoads];
#pragma unroll
    for (int i = 0; i < kLoads; ++i) {
        v[i] = __builtin_nontemporal_load(src + base + static_cast<size_t>(i) * kThreads);
    }
#pragma unroll
    for (int i = 0; i < kLoads; ++i) {
        __builtin_nontemporal_store(v[i], dst + base + static_cast<size_t>(i) * kThreads);
    }
}

// mismatches of dst against the byte value the source was filled with
__global__ __launch_bounds__(kThreads) void verify_kernel(const v4u *__restrict__ dst, unsigned fill, size_t n16,
                                                          unsigned long long *bad) {
    for (size_t j = static_cast<size_t>(blockIdx.x) * kThreads + threadIdx.x; j < n16;
         j += static_cast<size_t>(gridDim.x) * kThreads) {
        const v4u v = dst[j];
        if (v.x != fill || v.y != fill || v.z != fill || v.w != fill) {
            atomicAdd(bad, 1ull);
        }
    }
}

int main(int argc, char **argv) {
    const long mib = argc > 1 ? std::atol(argv[1]) : 1024;
    if (mib <= 0 || mib % 16 != 0 || mib > 65536) {
        std::fprintf(stderr, "hbm_rates: size must be a positive multiple of 16 MiB, at most 64 GiB\n");
        return 2;
    }
    const size_t bytes = static_cast<size_t>(mib) << 20;
    const size_t n16 = bytes / 16;
    const unsigned grid = static_cast<unsigned>(n16 / (kThreads * kLoads));  // exact: 16 MiB multiples
    v4u *a = nullptr, *b = nullptr;
    unsigned *sink = nullptr;
    unsigned long long *bad = nullptr;
    CHECK(hipMalloc(&a, bytes));
    CHECK(hipMalloc(&b, bytes));
    CHECK(hipMalloc(&sink, 64));
    CHECK(hipMalloc(&bad, sizeof(unsigned long long)));
    CHECK(hipMemset(a, 0x5a, bytes));
    CHECK(hipMemset(b, 0, bytes));
    CHECK(hipMemset(bad, 0, sizeof(unsigned long long)));
    CHECK(hipDeviceSynchronize());
    hipEvent_t e0, e1;
    CHECK(hipEventCreate(&e0));
    CHECK(hipEventCreate(&e1));
    auto median_ms = [&](auto launch) {
        for (int w = 0; w < 3; ++w) {
            launch();
        }
        CHECK(hipGetLastError());
        std::vector<float> t;
        for (int r = 0; r < 15; ++r) {
            CHECK(hipEventRecord(e0, 0));
            launch();
            CHECK(hipEventRecord(e1, 0));
            CHECK(hipEventSynchronize(e1));
            float ms = 0.0f;
            CHECK(hipEventElapsedTime(&ms, e0, e1));
            t.push_back(ms);
        }
        CHECK(hipGetLastError());
        std::sort(t.begin(), t.end());
        return static_cast<double>(t[t.size() / 2]);
    };
    const double read_ms = median_ms([&] { read_kernel<<<grid, kThreads>>>(a, sink); });
    const double write_ms = median_ms([&] { write_kernel<<<grid * kLoads, kThreads>>>(b); });
    const double copy_ms = median_ms([&] { copy_kernel<<<grid, kThreads>>>(a, b); });
    verify_kernel<<<2048, kThreads>>>(b, 0x5a5a5a5au, n16, bad);
    CHECK(hipGetLastError());
    unsigned long long mismatches = 0;
    CHECK(hipMemcpy(&mismatches, bad, sizeof(mismatches), hipMemcpyDeviceToHost));
    const double gb = static_cast<double>(bytes) / 1e9;
    std::printf("{\"bytes\": %zu, \"read_ms\": %.4f, \"read_GBs\": %.1f, \"write_ms\": %.4f, \"write_GBs\": %.1f, "
                "\"copy_ms\": %.4f, \"copy_GBs_read_plus_write\": %.1f, \"copy_ok\": %s}\n",
                bytes, read_ms, gb / (read_ms * 1e-3), write_ms, gb / (write_ms * 1e-3), copy_ms,
                2.0 * gb / (copy_ms * 1e-3), mismatches == 0 ? "true" : "false");
    CHECK(hipFree(a));
    CHECK(hipFree(b));
    CHECK(hipFree(sink));
    CHECK(hipFree(bad));
    return mismatches == 0 ? 0 : 1;
}
