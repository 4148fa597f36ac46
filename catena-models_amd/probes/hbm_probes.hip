// Two measurements behind the persistent decode step's design, on a resident
// grid shaped like the step's (one 512-thread block per CU):
//
//  burst    per iteration a grid barrier, then every wave loads K KB of one
//           of 16 cold 2 MiB regions (K 1 KB wave loads issued at once, like
//           the expert gate/up phase) and every block stamps its own end;
//           prints the spread of the barrier release and the distribution of
//           block completion times from the earliest start.
//  exchange per iteration one block writes W tagged 64-bit words (a row of
//           the step's exchange) after every other block is already polling
//           them the way the step does (each thread its words, re-polling
//           the missing ones); prints how long after the write the median
//           and the last block see the whole row.
//
// Build and run (hipcc, gfx950):
//   hipcc --offload-arch=gfx950 -O3 -o hbm_probes catena-models_amd/probes/hbm_probes.hip
//   ./hbm_probes
// Every wait is bounded; a wait that runs out sets an error flag that is
// printed with the results. Needs about 16.2 GiB of device memory.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdint>
#include <cstdio>
#include <vector>

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

#define CHECK(x)                                                               \
  do {                                                                         \
    hipError_t e_ = (x);                                                       \
    if (e_ != hipSuccess) {                                                    \
      printf("%s failed: %s\n", #x, hipGetErrorString(e_));                    \
      return 1;                                                                \
    }                                                                          \
  } while (0)

__device__ bool grid_barrier(unsigned* count, unsigned* gen, unsigned nblocks, unsigned* err) {
  __syncthreads();
  bool ok = true;
  if (threadIdx.x == 0) {
    const unsigned g = __hip_atomic_load(gen, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const unsigned arrived = __hip_atomic_fetch_add(count, 1u, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
    if (arrived == nblocks - 1) {
      __hip_atomic_store(count, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      __hip_atomic_store(gen, g + 1, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_AGENT);
    } else {
      unsigned spins = 0;
      while (__hip_atomic_load(gen, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_AGENT) == g) {
        if (++spins > (1u << 24)) {
          __hip_atomic_store(err, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          ok = false;
          break;
        }
      }
    }
  }
  __syncthreads();
  return ok;
}

// ------------------------------------------------------------------ burst

template <int K>
__global__ __launch_bounds__(512) void burst(const u32x4* __restrict__ base, const uint64_t* __restrict__ regions,
                                             int iters, unsigned* bar, uint64_t* st, unsigned* err,
                                             uint32_t* sink) {
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  uint32_t acc = 0;
  for (int it = 0; it < iters; ++it) {
    if (!grid_barrier(bar, bar + 32, gridDim.x, err)) return;
    const uint64_t t0 = __builtin_amdgcn_s_memrealtime();
    const int gw = blockIdx.x * 8 + wave;
    const u32x4* rb = base + regions[it * 16 + gw % 16] / 16;
    const int within = gw / 16;
    u32x4 v[K];
#pragma unroll
    for (int k = 0; k < K; ++k) v[k] = rb[((size_t)within * K + k) * 64 + lane];
#pragma unroll
    for (int k = 0; k < K; ++k) acc += v[k].x ^ v[k].y ^ v[k].z ^ v[k].w;
    __syncthreads();
    const uint64_t t1 = __builtin_amdgcn_s_memrealtime();
    if (threadIdx.x == 0) {
      st[((size_t)it * gridDim.x + blockIdx.x) * 2] = t0;
      st[((size_t)it * gridDim.x + blockIdx.x) * 2 + 1] = t1;
    }
  }
  if (acc == 0x12345678u) sink[0] = acc;  // keeps the loads
}

// --------------------------------------------------------------- exchange

__device__ __forceinline__ uint64_t word_load(const uint64_t* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

template <int MAXW>
__global__ __launch_bounds__(512) void exchange(uint64_t* words, int W, int iters, uint64_t* st, unsigned* err,
                                                unsigned* bar) {
  const int G = gridDim.x;
  for (int it = 0; it < iters; ++it) {
    if (!grid_barrier(bar, bar + 32, G, err)) return;
    const uint32_t tag = 1000 + it;
    const int src = it % G;
    if ((int)blockIdx.x == src) {
      // let every other block reach its poll first (the barrier release is skewed)
      const uint64_t t_start = __builtin_amdgcn_s_memrealtime();
      while (__builtin_amdgcn_s_memrealtime() - t_start < 1500) {
      }
      const uint64_t t = __builtin_amdgcn_s_memrealtime();
      if (threadIdx.x == 0) st[(size_t)it * (G + 1) + G] = t;
      for (int i = threadIdx.x; i < W; i += 512)
        __hip_atomic_store(words + i, ((uint64_t)tag << 32) | (uint32_t)i, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    } else {
      uint64_t v[MAXW];
#pragma unroll
      for (int j = 0; j < MAXW; ++j) v[j] = word_load(words + min((int)threadIdx.x + 512 * j, W - 1));
      unsigned spins = 0;
      bool ok = true;
      while (true) {
        bool ready = true;
#pragma unroll
        for (int j = 0; j < MAXW; ++j) ready &= (uint32_t)(v[j] >> 32) == tag;
        if (ready) break;
        if (++spins > (1u << 22)) {
          __hip_atomic_store(err, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          ok = false;
          break;
        }
#pragma unroll
        for (int j = 0; j < MAXW; ++j)
          if ((uint32_t)(v[j] >> 32) != tag) v[j] = word_load(words + min((int)threadIdx.x + 512 * j, W - 1));
      }
      __syncthreads();
      if (!ok) return;
      if (threadIdx.x == 0) st[(size_t)it * (G + 1) + blockIdx.x] = __builtin_amdgcn_s_memrealtime();
    }
  }
}

int main() {
  int grid = 0;
  CHECK(hipDeviceGetAttribute(&grid, hipDeviceAttributeMultiprocessorCount, 0));
  if (grid > 256) {  // the burst regions hold 16 KB x 8 waves x grid / 16 <= 4 MiB at 32 KB per wave
    printf("the probe assumes at most 256 CUs (this device has %d)\n", grid);
    return 1;
  }
  const size_t buf = (size_t)16 << 30;
  char* base = nullptr;
  CHECK(hipMalloc(&base, buf));
  CHECK(hipMemset(base, 1, buf));
  const int iters = 48;
  uint64_t *regions, *st;
  unsigned *bar, *err;
  uint32_t* sink;
  uint64_t* words;
  CHECK(hipMalloc(&regions, iters * 16 * 8));
  CHECK(hipMalloc(&st, (size_t)200 * (grid + 1) * 16));
  CHECK(hipMalloc(&bar, 256));
  CHECK(hipMalloc(&err, 4));
  CHECK(hipMalloc(&sink, 4));
  CHECK(hipMalloc(&words, 2048 * 8));
  printf("%d blocks x 512 threads\n\nburst: K KB per wave from 16 cold 2 MiB regions, times from the earliest start (us)\n",
         grid);
  const uint64_t slot = 4ull << 20, nslots = buf / slot;
  int salt = 1;
  auto run_burst = [&](const char* name, auto kernel, double mb) -> int {
    std::vector<uint64_t> reg(iters * 16);
    for (int it = 0; it < iters; ++it)
      for (int r = 0; r < 16; ++r) reg[it * 16 + r] = ((uint64_t)(it * 16 + r + 977 * salt) * 7919u % nslots) * slot;
    ++salt;
    CHECK(hipMemcpy(regions, reg.data(), reg.size() * 8, hipMemcpyHostToDevice));
    CHECK(hipMemset(bar, 0, 256));
    CHECK(hipMemset(err, 0, 4));
    hipLaunchKernelGGL(kernel, dim3(grid), dim3(512), 0, 0, (const u32x4*)base, regions, iters, bar, st, err, sink);
    CHECK(hipDeviceSynchronize());
    unsigned e = 0;
    CHECK(hipMemcpy(&e, err, 4, hipMemcpyDeviceToHost));
    std::vector<uint64_t> h((size_t)iters * grid * 2);
    CHECK(hipMemcpy(h.data(), st, h.size() * 8, hipMemcpyDeviceToHost));
    double skew = 0, p[5] = {0, 0, 0, 0, 0};
    int n = 0;
    for (int it = 4; it < iters; ++it, ++n) {
      uint64_t t0 = ~0ull, t0max = 0;
      for (int b = 0; b < grid; ++b) {
        t0 = std::min(t0, h[((size_t)it * grid + b) * 2]);
        t0max = std::max(t0max, h[((size_t)it * grid + b) * 2]);
      }
      std::vector<double> ends(grid);
      for (int b = 0; b < grid; ++b) ends[b] = (h[((size_t)it * grid + b) * 2 + 1] - t0) * 0.01;
      std::sort(ends.begin(), ends.end());
      skew += (t0max - t0) * 0.01;
      p[0] += ends[0];
      p[1] += ends[grid / 10];
      p[2] += ends[grid / 2];
      p[3] += ends[grid * 9 / 10];
      p[4] += ends[grid - 1];
    }
    printf("%-28s err %u: release spread %5.2f | block end min %5.2f p10 %5.2f p50 %5.2f p90 %5.2f max %5.2f\n", name,
           e, skew / n, p[0] / n, p[1] / n, p[2] / n, p[3] / n, p[4] / n);
    (void)mb;
    return 0;
  };
  if (run_burst("1 KB x 8 waves (2.1 MB)", burst<1>, 2.1)) return 1;
  if (run_burst("4 KB x 8 waves (8.4 MB)", burst<4>, 8.4)) return 1;
  if (run_burst("8 KB x 8 waves (16.8 MB)", burst<8>, 16.8)) return 1;
  if (run_burst("16 KB x 8 waves (33.6 MB)", burst<16>, 33.6)) return 1;
  if (run_burst("32 KB x 8 waves (67.1 MB)", burst<32>, 67.1)) return 1;

  printf("\nexchange: one block writes a row of W tagged words, every other block polls it (us after the write)\n");
  const int xiters = 200;
  auto run_exchange = [&](const char* name, auto kernel, int W) -> int {
    CHECK(hipMemset(words, 0, 2048 * 8));
    CHECK(hipMemset(err, 0, 4));
    CHECK(hipMemset(bar, 0, 256));
    CHECK(hipMemset(st, 0, (size_t)xiters * (grid + 1) * 8));
    hipLaunchKernelGGL(kernel, dim3(grid), dim3(512), 0, 0, words, W, xiters, st, err, bar);
    CHECK(hipDeviceSynchronize());
    unsigned e = 0;
    CHECK(hipMemcpy(&e, err, 4, hipMemcpyDeviceToHost));
    std::vector<uint64_t> h((size_t)xiters * (grid + 1));
    CHECK(hipMemcpy(h.data(), st, h.size() * 8, hipMemcpyDeviceToHost));
    double p50 = 0, last = 0;
    int n = 0;
    for (int it = 8; it < xiters; ++it, ++n) {
      const double tw = (double)h[(size_t)it * (grid + 1) + grid];
      std::vector<double> d;
      for (int b = 0; b < grid; ++b)
        if (b != it % grid) d.push_back(((double)h[(size_t)it * (grid + 1) + b] - tw) * 0.01);
      std::sort(d.begin(), d.end());
      p50 += d[d.size() / 2];
      last += d.back();
    }
    printf("%-28s err %u: median block %5.2f, last block %5.2f\n", name, e, p50 / n, last / n);
    return 0;
  };
  if (run_exchange("1 word", exchange<1>, 1)) return 1;
  if (run_exchange("1024 words (8 KB)", exchange<2>, 1024)) return 1;
  if (run_exchange("2048 words (16 KB)", exchange<4>, 2048)) return 1;
  return 0;
}
