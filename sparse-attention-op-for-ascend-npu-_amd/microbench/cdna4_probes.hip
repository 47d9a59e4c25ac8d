// Hardware probes behind the attention kernel's design (MI355X / gfx950).
//
// Three measurements, each over 256 workgroups (one per CU) and printed as one
// table row per configuration:
//  1. L2 -> CU bandwidth of LDS DMA (buffer_load ... lds, 1 KB per
//     instruction) against the number of instructions each wave keeps in
//     flight, with 8 and 4 waves per CU.  The source is a 2 MB buffer, so
//     every load after the first pass hits L2.
//  2. LDS read bandwidth of 4 reader waves (the K operand read ds_read_b128,
//     the V operand read ds_read_b64_tr_b16) alone and while 4 other waves of
//     the workgroup stream LDS DMA or VGPR loads.
//  3. MFMA issue (v_mfma_f32_32x32x16_bf16, two independent accumulators)
//     with n independent VALU instructions (v_exp_f32 or v_fma_f32) after
//     each MFMA, at 1 and 2 waves per SIMD: time per MFMA per SIMD.
//
// Build and run: python -m trianglemix.microbench  (or hipcc --offload-arch=gfx950 -O3 this file).

#include <hip/hip_runtime.h>

#include <cstdio>
#include <cstdlib>

namespace {

#define CHECK(x)                                                                  \
  do {                                                                            \
    hipError_t e_ = (x);                                                          \
    if (e_ != hipSuccess) {                                                       \
      std::fprintf(stderr, "%s failed: %s\n", #x, hipGetErrorString(e_));         \
      std::exit(1);                                                               \
    }                                                                             \
  } while (0)

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef short i16x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
#define LDS_PTR(p) ((__attribute__((address_space(3))) void*)(p))

constexpr int kCUs = 256;
constexpr unsigned kSourceBytes = 2u << 20;  // L2-resident source
constexpr int kLdsBytes = 131072;

// ---- 1. L2 -> CU: each wave keeps `depth` 1 KB loads in flight, then waits for all of them.
template <bool kToLds, int kDepth>
__global__ void __launch_bounds__(512) memory_path(const char* src, float* sink, int rounds) {
  __shared__ __attribute__((aligned(1024))) char lds[kLdsBytes];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int waves = blockDim.x >> 6;
  const __amdgpu_buffer_rsrc_t r = __builtin_amdgcn_make_buffer_rsrc((void*)src, (short)0, kSourceBytes + 1024,
                                                                      0x00020000);
  f32x4 acc = {0, 0, 0, 0};
  for (int round = 0; round < rounds; ++round) {
#pragma unroll
    for (int j = 0; j < kDepth; ++j) {
      // each wave streams through the buffer from its own start, never re-reading a KB it read in the last 2 MB
      // (no L1 reuse); + lane * 16 stays inside the 1 KB
      const unsigned off = ((unsigned)(blockIdx.x * waves + wave) * 65536u + ((unsigned)round * kDepth + j) * 1024u) &
                           (kSourceBytes - 1);
      if constexpr (kToLds) {
        char* dst = lds + ((wave * 16 + j) & 127) * 1024;  // 1 KB per instruction, inside the 128 KB
        asm volatile("" : "+s"(dst));
        __builtin_amdgcn_raw_ptr_buffer_load_lds(r, LDS_PTR(dst), 16, (unsigned)(lane * 16), off, 0, 0);
      } else {
        acc += __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(r, (unsigned)(lane * 16), off, 0));
      }
    }
    __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
  }
  __syncthreads();
  sink[blockIdx.x * blockDim.x + threadIdx.x] = reinterpret_cast<float*>(lds)[threadIdx.x] + acc[0] + acc[3];
}

// ---- 2. LDS reads (waves 0-3) against loads by waves 4-7.
// kRead: 1 = ds_read_b128 (K pattern), 2 = ds_read_b64_tr_b16 (V pattern); kLoad: 0 none, 1 LDS DMA, 2 VGPR loads.
template <int kRead, int kLoad>
__global__ void __launch_bounds__(512) lds_mix(const char* src, float* sink, unsigned long long* ticks, int rounds) {
  __shared__ __attribute__((aligned(1024))) char lds[kLdsBytes];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  for (int i = threadIdx.x; i < kLdsBytes / 4; i += blockDim.x) reinterpret_cast<float*>(lds)[i] = 0.0f;
  __syncthreads();
  const __amdgpu_buffer_rsrc_t r = __builtin_amdgcn_make_buffer_rsrc((void*)src, (short)0, kSourceBytes + 1024,
                                                                      0x00020000);
  f32x4 acc = {0, 0, 0, 0};
  const unsigned long long t0 = __builtin_amdgcn_s_memrealtime();
  if (wave < 4) {
    if constexpr (kRead == 1) {
      const int row = lane & 31, half = lane >> 5;
      unsigned addr[8];
      for (int c = 0; c < 8; ++c)  // swizzled 16-byte chunk of a 32-row x 256 B tile: < 32 KB
        addr[c] = (unsigned)(size_t)LDS_PTR(lds + wave * 8192 + row * 256 + 16 * ((2 * c + half) ^ (row & 15)));
      for (int round = 0; round < rounds; ++round) {
#pragma unroll
        for (int c = 0; c < 8; ++c) {
          f32x4 x;
          asm volatile("ds_read_b128 %0, %1" : "=v"(x) : "v"(addr[c]) : "memory");
          acc += x;
        }
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
      }
    } else if constexpr (kRead == 2) {
      const int key = 4 * (lane >> 5) + ((lane & 15) >> 2);
      unsigned addr[4];
      for (int m = 0; m < 4; ++m) {  // highest byte read: 3 * 8192 + 7 * 256 + 255 + 6144 + 8 < 32 KB
        const int d = 32 * m + 16 * ((lane >> 4) & 1) + 4 * (lane & 3);
        addr[m] = (unsigned)(size_t)LDS_PTR(lds + wave * 8192 + key * 256 + 16 * ((d >> 3) ^ ((key & 3) << 2)) +
                                            2 * (d & 7));
      }
      for (int round = 0; round < rounds; ++round) {
#pragma unroll
        for (int k = 0; k < 8; ++k) {
          i16x4 lo, hi;
          asm volatile("ds_read_b64_tr_b16 %0, %1 offset:%2" : "=v"(lo) : "v"(addr[k & 3]), "i"(16 * (k >> 2) * 256)
                       : "memory");
          asm volatile("ds_read_b64_tr_b16 %0, %1 offset:%2" : "=v"(hi) : "v"(addr[k & 3]),
                       "i"(16 * (k >> 2) * 256 + 2048) : "memory");
          acc[0] += (float)lo[0] + (float)hi[1];
        }
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
      }
    }
  } else if constexpr (kLoad != 0) {
    for (int round = 0; round < rounds; ++round) {
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const unsigned off = ((unsigned)(blockIdx.x * 8 + wave) * 65536u + ((unsigned)round * 8 + j) * 1024u) &
                             (kSourceBytes - 1);
        if constexpr (kLoad == 1) {
          char* dst = lds + 65536 + ((wave - 4) * 8 + j) * 1024;  // 32 KB above the readers' area
          asm volatile("" : "+s"(dst));
          __builtin_amdgcn_raw_ptr_buffer_load_lds(r, LDS_PTR(dst), 16, (unsigned)(lane * 16), off, 0, 0);
        } else {
          acc += __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(r, (unsigned)(lane * 16), off, 0));
        }
      }
      __builtin_amdgcn_s_waitcnt(0x0F70);
    }
  }
  const unsigned long long t1 = __builtin_amdgcn_s_memrealtime();
  if (lane == 0 && blockIdx.x == 0) ticks[wave] = t1 - t0;
  __syncthreads();
  sink[blockIdx.x * blockDim.x + threadIdx.x] = reinterpret_cast<float*>(lds)[threadIdx.x] + acc[0] + acc[3];
}

// ---- 3. MFMA with n independent VALU instructions after each one.
template <int kValu, bool kExp>
__global__ void __launch_bounds__(512) mfma_valu(float* sink, int rounds) {
  bf16x8 a, b;
  for (int i = 0; i < 8; ++i) {
    a[i] = (__bf16)(threadIdx.x * 0.001f + i);
    b[i] = (__bf16)(i * 0.5f);
  }
  f32x16 acc0 = {}, acc1 = {};
  float x[12];
  for (int i = 0; i < 12; ++i) x[i] = threadIdx.x * 1e-3f + i;
  for (int round = 0; round < rounds; ++round) {
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      if (k & 1) {
        acc1 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, acc1, 0, 0, 0);
      } else {
        acc0 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, acc0, 0, 0, 0);
      }
#pragma unroll
      for (int v = 0; v < kValu; ++v) {
        if constexpr (kExp) {
          asm volatile("v_exp_f32 %0, %0" : "+v"(x[v]));
        } else {
          asm volatile("v_fma_f32 %0, %0, %0, 1.0" : "+v"(x[v]));
        }
      }
      __builtin_amdgcn_sched_barrier(0);
    }
  }
  float s = 0.0f;
  for (int i = 0; i < 16; ++i) s += acc0[i] + acc1[i];
  for (int i = 0; i < 12; ++i) s += x[i];
  sink[blockIdx.x * blockDim.x + threadIdx.x] = s;
}

struct Timer {
  hipEvent_t start, stop;
  Timer() {
    CHECK(hipEventCreate(&start));
    CHECK(hipEventCreate(&stop));
  }
  ~Timer() {
    (void)hipEventDestroy(start);
    (void)hipEventDestroy(stop);
  }
  template <typename F>
  float ms(F launch) {  // one untimed launch, then one timed
    launch();
    CHECK(hipGetLastError());
    CHECK(hipEventRecord(start));
    launch();
    CHECK(hipEventRecord(stop));
    CHECK(hipEventSynchronize(stop));
    float t = 0.0f;
    CHECK(hipEventElapsedTime(&t, start, stop));
    return t;
  }
};

template <bool kToLds, int kDepth>
void probe_memory_path(const char* src, float* sink, int threads) {
  const int rounds = 4000 / kDepth;
  Timer t;
  const float ms = t.ms([&] { hipLaunchKernelGGL((memory_path<kToLds, kDepth>), dim3(kCUs), dim3(threads), 0, 0,
                                                 src, sink, rounds); });
  const double bytes_per_cu = double(threads / 64) * rounds * kDepth * 1024;
  std::printf("l2_to_cu   %-9s waves/CU %d  in flight/wave %2d  %7.1f GB/s per CU  (%.0f TB/s chip)\n",
              kToLds ? "lds-dma" : "vgpr-load", threads / 64, kDepth, bytes_per_cu / (ms * 1e6),
              bytes_per_cu * kCUs / (ms * 1e-3) / 1e12);
}

template <int kRead, int kLoad>
void probe_lds_mix(const char* src, float* sink, unsigned long long* ticks) {
  const int rounds = 2000;
  Timer t;
  (void)t.ms([&] { hipLaunchKernelGGL((lds_mix<kRead, kLoad>), dim3(kCUs), dim3(512), 0, 0, src, sink, ticks,
                                      rounds); });
  unsigned long long h[8] = {};
  CHECK(hipMemcpy(h, ticks, sizeof(h), hipMemcpyDeviceToHost));
  const double bytes = 4.0 * rounds * 8 * 1024;  // per CU and role
  const char* reads[] = {"-", "ds_read_b128", "ds_read_b64_tr"};
  const char* loads[] = {"-", "lds-dma", "vgpr-load"};
  std::printf("lds_mix    reads %-15s + loads %-9s: reads %6.1f GB/s per CU, loads %6.1f GB/s per CU\n",
              reads[kRead], loads[kLoad], kRead ? bytes / (h[0] * 10.0) : 0.0, kLoad ? bytes / (h[4] * 10.0) : 0.0);
}

template <int kValu, bool kExp>
void probe_mfma_valu(float* sink, int threads) {
  const int rounds = 200;
  Timer t;
  const float ms = t.ms([&] { hipLaunchKernelGGL((mfma_valu<kValu, kExp>), dim3(kCUs), dim3(threads), 0, 0, sink,
                                                 rounds); });
  const double mfma_per_simd = rounds * 8.0 * (threads / 64 / 4);
  std::printf("mfma_valu  waves/SIMD %d  + %2d %s per MFMA: %6.2f ns per MFMA per SIMD\n", threads / 256, kValu,
              kExp ? "v_exp_f32" : "v_fma_f32", ms * 1e6 / mfma_per_simd);
}

}  // namespace

int main() {
  char* src = nullptr;
  float* sink = nullptr;
  unsigned long long* ticks = nullptr;
  CHECK(hipMalloc(&src, kSourceBytes + 1024));
  CHECK(hipMalloc(&sink, kCUs * 512 * sizeof(float)));
  CHECK(hipMalloc(&ticks, 8 * sizeof(unsigned long long)));
  CHECK(hipMemset(src, 0, kSourceBytes + 1024));
  for (int threads : {512, 256}) {
    probe_memory_path<true, 1>(src, sink, threads);
    probe_memory_path<true, 4>(src, sink, threads);
    probe_memory_path<true, 8>(src, sink, threads);
    probe_memory_path<true, 16>(src, sink, threads);
  }
  probe_lds_mix<1, 0>(src, sink, ticks);
  probe_lds_mix<2, 0>(src, sink, ticks);
  probe_lds_mix<0, 1>(src, sink, ticks);
  probe_lds_mix<1, 1>(src, sink, ticks);
  probe_lds_mix<2, 1>(src, sink, ticks);
  probe_lds_mix<1, 2>(src, sink, ticks);
  for (int threads : {256, 512}) {
    probe_mfma_valu<0, true>(sink, threads);
    probe_mfma_valu<2, true>(sink, threads);
    probe_mfma_valu<4, true>(sink, threads);
    probe_mfma_valu<8, true>(sink, threads);
    probe_mfma_valu<4, false>(sink, threads);
    probe_mfma_valu<8, false>(sink, threads);
  }
  CHECK(hipFree(src));
  CHECK(hipFree(sink));
  CHECK(hipFree(ticks));
  return 0;
}
