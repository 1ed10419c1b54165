// Practical HBM ceilings for the traffic shapes of the bench workloads, on the GPU it runs on:
// minimal streaming kernels (16-byte non-temporal loads and stores, nothing else) moving the
// same bytes as a workload, timed with HIP events over back-to-back launches that rotate over
// buffer sets larger than the 256 MB MALL.  Prints one JSON object:
//   r2w1_cfg3: read 134,217,728 B + write 67,108,864 B per launch (configs[2]'s K/V in, codes out)
//   r2w1_cfg4: read  67,108,864 B + write 33,554,432 B per launch (configs[3]'s rows in, codes out)
//   copy_1to1: read 134,217,728 B + write 134,217,728 B per launch
// each as {"us": per-launch time, "GB_s": bytes / time}.  Run by bench.py (measurement only).
#include <hip/hip_runtime.h>

#include <cstdio>
#include <vector>

namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

// 16 bytes in, 8 bytes out per thread
__global__ __launch_bounds__(256) void read2_write1(const u32x4* __restrict__ in,
                                                     u32x2* __restrict__ out, int64_t n16) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= n16) return;
  const u32x4 v = __builtin_nontemporal_load(in + i);
  u32x2 o;
  o[0] = v[0] ^ v[1];
  o[1] = v[2] ^ v[3];
  __builtin_nontemporal_store(o, out + i);
}

__global__ __launch_bounds__(256) void copy16(const u32x4* __restrict__ in, u32x4* __restrict__ out,
                                              int64_t n16) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= n16) return;
  __builtin_nontemporal_store(__builtin_nontemporal_load(in + i), out + i);
}

}  // namespace

int main() {
  const int64_t big = 134217728;  // bytes read per configs[2]-shaped launch
  const int sets = 8;             // 8 x (128 + 128) MB rotated
  std::vector<u32x4*> in(sets), out(sets);
  for (int s = 0; s < sets; ++s) {
    if (hipMalloc(&in[s], big) != hipSuccess || hipMalloc(&out[s], big) != hipSuccess ||
        hipMemset(in[s], 1, big) != hipSuccess) {
      std::printf("{\"error\": \"device setup failed\"}\n");
      return 2;
    }
  }
  hipEvent_t a, b;
  if (hipEventCreate(&a) != hipSuccess || hipEventCreate(&b) != hipSuccess) return 2;
  auto time_us = [&](auto launch) -> double {
    for (int w = 0; w < 200; ++w) launch(w % sets);
    if (hipDeviceSynchronize() != hipSuccess) return -1.0;
    const int reps = 800;
    if (hipEventRecord(a) != hipSuccess) return -1.0;
    for (int r = 0; r < reps; ++r) launch(r % sets);
    if (hipEventRecord(b) != hipSuccess || hipEventSynchronize(b) != hipSuccess) return -1.0;
    float ms = 0.0f;
    if (hipEventElapsedTime(&ms, a, b) != hipSuccess) return -1.0;
    return ms * 1e3 / reps;
  };
  auto r2w1 = [&](int64_t in_bytes) {
    const int64_t n16 = in_bytes / 16;
    const dim3 grid((unsigned)((n16 + 255) / 256)), block(256);
    return time_us([&](int s) {
      read2_write1<<<grid, block>>>(in[s], reinterpret_cast<u32x2*>(out[s]), n16);
    });
  };
  const double t3 = r2w1(big), t4 = r2w1(big / 2);
  const int64_t n16 = big / 16;
  const double tc = time_us([&](int s) {
    copy16<<<dim3((unsigned)((n16 + 255) / 256)), dim3(256)>>>(in[s], out[s], n16);
  });
  if (t3 <= 0 || t4 <= 0 || tc <= 0) {
    std::printf("{\"error\": \"kernel failed\"}\n");
    return 3;
  }
  std::printf("{\"r2w1_cfg3\": {\"us\": %.2f, \"GB_s\": %.1f}, \"r2w1_cfg4\": {\"us\": %.2f, "
              "\"GB_s\": %.1f}, \"copy_1to1\": {\"us\": %.2f, \"GB_s\": %.1f}}\n",
              t3, 1.5 * big / t3 / 1e3, t4, 0.75 * big / t4 / 1e3, tc, 2.0 * big / tc / 1e3);
  return 0;
}
