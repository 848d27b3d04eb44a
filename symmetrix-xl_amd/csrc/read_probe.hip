// HBM read-rate probe: the reference rates for the message gather
// (gather_messages_kernel in layers.hip), measured on the device it runs on.
//
//   read_probe [MiB]      (default 756, the medium workload's message bytes)
//
// 1. stream: every float4 of a MiB-sized buffer read once, grid-stride, one
//    float per workgroup written -- the plain read rate;
// 2. rows: the gather's access pattern without its bookkeeping -- the buffer
//    cut into 2 KiB rows, each workgroup of 128 threads summing 74 rows taken
//    in a fixed random order (8 in flight per thread) and writing one 2 KiB
//    row -- the rate a per-source sum of scattered message rows can reach.
// Each is timed with HIP events over 20 launches after 3 warmups; prints one
// line per pattern in GB/s (10^9 bytes read per second).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdio>
#include <cstdlib>
#include <numeric>
#include <random>
#include <vector>

namespace {

#define CHECK(x)                                                                         \
    do {                                                                                 \
        hipError_t err_ = (x);                                                           \
        if (err_ != hipSuccess) {                                                        \
            std::fprintf(stderr, "%s: %s\n", #x, hipGetErrorString(err_));               \
            std::exit(1);                                                                \
        }                                                                                \
    } while (0)

__global__ void __launch_bounds__(256) stream_kernel(const float4* __restrict__ in, size_t n, float* __restrict__ out)
{
    float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
    for (size_t i = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n;
         i += static_cast<size_t>(gridDim.x) * blockDim.x) {
        const float4 v = in[i];
        acc.x += v.x, acc.y += v.y, acc.z += v.z, acc.w += v.w;
    }
    const float s = acc.x + acc.y + acc.z + acc.w;
    if (threadIdx.x == 0 || s == 1.0e30f) out[blockIdx.x] = s;
}

constexpr int kRow4 = 128;       // float4 per 2 KiB row
constexpr int kRowsPerGroup = 74;
constexpr int kInFlight = 8;

__global__ void __launch_bounds__(128) rows_kernel(const float4* __restrict__ in, const int* __restrict__ order,
                                                   float4* __restrict__ out)
{
    const int* rows = order + static_cast<size_t>(blockIdx.x) * kRowsPerGroup;
    float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
    for (int r = 0; r < kRowsPerGroup; r += kInFlight) {
        float4 v[kInFlight];
#pragma unroll
        for (int u = 0; u < kInFlight; ++u) {
            v[u] = make_float4(0.f, 0.f, 0.f, 0.f);
            if (r + u < kRowsPerGroup) v[u] = in[static_cast<size_t>(rows[r + u]) * kRow4 + threadIdx.x];
        }
#pragma unroll
        for (int u = 0; u < kInFlight; ++u) acc.x += v[u].x, acc.y += v[u].y, acc.z += v[u].z, acc.w += v[u].w;
    }
    out[static_cast<size_t>(blockIdx.x) * kRow4 + threadIdx.x] = acc;
}

template <class Launch>
double time_ms(Launch launch)
{
    hipEvent_t a, b;
    CHECK(hipEventCreate(&a));
    CHECK(hipEventCreate(&b));
    for (int i = 0; i < 3; ++i) launch();
    CHECK(hipDeviceSynchronize());
    CHECK(hipEventRecord(a, nullptr));
    for (int i = 0; i < 20; ++i) launch();
    CHECK(hipEventRecord(b, nullptr));
    CHECK(hipEventSynchronize(b));
    float ms = 0.f;
    CHECK(hipEventElapsedTime(&ms, a, b));
    CHECK(hipEventDestroy(a));
    CHECK(hipEventDestroy(b));
    return ms / 20.0;
}

}  // namespace

int main(int argc, char** argv)
{
    const size_t mib = argc > 1 ? std::strtoull(argv[1], nullptr, 10) : 756;
    const size_t bytes = mib << 20;
    const size_t n4 = bytes / sizeof(float4);
    float4* in = nullptr;
    CHECK(hipMalloc(&in, bytes));
    CHECK(hipMemset(in, 0, bytes));
    int cus = 0;
    CHECK(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, 0));

    const int stream_blocks = cus * 16;
    float* partial = nullptr;
    CHECK(hipMalloc(&partial, stream_blocks * sizeof(float)));
    const double t_stream =
        time_ms([&] { stream_kernel<<<stream_blocks, 256>>>(in, n4, partial); });
    std::printf("stream: %zu MiB read in %.4f ms = %.0f GB/s\n", mib, t_stream, bytes / (t_stream * 1e-3) / 1e9);

    const size_t rows = n4 / kRow4;
    const size_t groups = rows / kRowsPerGroup;
    std::vector<int> order(groups * kRowsPerGroup);
    std::iota(order.begin(), order.end(), 0);
    std::shuffle(order.begin(), order.end(), std::mt19937(7));
    int* d_order = nullptr;
    float4* out = nullptr;
    CHECK(hipMalloc(&d_order, order.size() * sizeof(int)));
    CHECK(hipMemcpy(d_order, order.data(), order.size() * sizeof(int), hipMemcpyHostToDevice));
    CHECK(hipMalloc(&out, groups * kRow4 * sizeof(float4)));
    const double t_rows =
        time_ms([&] { rows_kernel<<<static_cast<int>(groups), 128>>>(in, d_order, out); });
    const double row_bytes = static_cast<double>(order.size()) * kRow4 * sizeof(float4);
    std::printf("rows: %zu groups of %d random 2 KiB rows (%.0f MiB) in %.4f ms = %.0f GB/s read\n", groups,
                kRowsPerGroup, row_bytes / (1 << 20), t_rows, row_bytes / (t_rows * 1e-3) / 1e9);
    CHECK(hipFree(in));
    CHECK(hipFree(partial));
    CHECK(hipFree(d_order));
    CHECK(hipFree(out));
    return 0;
}
