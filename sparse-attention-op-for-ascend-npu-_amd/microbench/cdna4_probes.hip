// Hardware probes behind the attention kernel's design (MI355X / gfx950).
//
// Six measurements, each over 256 workgroups (one per CU) and printed as one
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
//  4. The attention loop body (one 32-key tile per wave and iteration: K
//     reads, the QK^T chain, exponentials, row sum and max, V transposed
//     reads, PV into four accumulators, 1 KB of LDS DMA per MFMA step and a
//     barrier per iteration -- the kernel's KV-quarter shape, 8 waves per CU)
//     and the same work as 4 waves of two heads each (every K/V read feeds
//     two MFMAs, one wave per SIMD).  K/V come from an L2-resident buffer of
//     zeros or of random bf16 values; each row gives the time per iteration,
//     the shader clock over the launch (s_memtime against the 100 MHz
//     s_memrealtime) and the cycles per iteration.
//  5. MFMA alone at full load: back-to-back v_mfma_f32_32x32x16_bf16 into
//     four independent accumulators, operands read once from the zero or
//     random buffer, at 1 and 2 waves per SIMD.  Each row gives the MFMA
//     rate as chip TFLOP/s and as a fraction of the 2.5 PFLOP/s bf16 peak
//     (32 cycles per MFMA at 2.4 GHz), beside the shader clock: the power
//     limit sets the clock, so it is the chip's sustainable MFMA rate for
//     such operands.
//  6. The launch floor: 16 launches of a kernel that does next to nothing
//     (one LDS round trip and one 4-byte store per thread), back to back on
//     one stream and as one HIP graph, in the attention kernel's workgroup
//     shape (512 threads, 144 KB of LDS) and in a light one (64 threads,
//     4 KB).  Each row gives the time per launch: the dispatch ramp, the
//     drain and the gap between launches that any kernel of that shape pays.
//
// Build and run: python -m trianglemix.microbench  (or hipcc --offload-arch=gfx950 -O3 this file).

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdio>
#include <cstdlib>
#include <cstring>

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

// ---- 6. Launch floor: one LDS round trip and one store per thread.
template <int kLdsBytes, int kThreads>
__global__ void __launch_bounds__(kThreads) launch_floor(float* sink) {
  __shared__ float buf[kLdsBytes / 4];
  buf[threadIdx.x] = float(threadIdx.x);
  __syncthreads();
  sink[blockIdx.x * 512 + threadIdx.x] = buf[(threadIdx.x + 1) % kThreads];
}

// ---- 5. MFMA alone: eight operand pairs per lane (distinct per lane and wave) feed four accumulators.
__global__ void __launch_bounds__(512) mfma_power(const bf16x8* src, float* sink, int rounds,
                                                  unsigned long long* clocks) {
  const unsigned long long c0 = __builtin_amdgcn_s_memtime(), r0 = __builtin_amdgcn_s_memrealtime();
  // 16 operands of 16 B per lane from a 4096-lane window of the source: at most 65,536 of its 131,136.
  const bf16x8* mine = src + ((blockIdx.x * blockDim.x + threadIdx.x) % 4096) * 16;
  bf16x8 a[8], b[8];
#pragma unroll
  for (int k = 0; k < 8; ++k) {
    a[k] = mine[k];
    b[k] = mine[8 + k];
  }
  f32x16 acc[4] = {};
  for (int round = 0; round < rounds; ++round) {
#pragma unroll
    for (int k = 0; k < 8; ++k) acc[k & 3] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[k], b[k], acc[k & 3], 0, 0, 0);
  }
  float s = 0.0f;
#pragma unroll
  for (int m = 0; m < 4; ++m) {
#pragma unroll
    for (int i = 0; i < 16; ++i) s += acc[m][i];
  }
  sink[blockIdx.x * blockDim.x + threadIdx.x] = s;
  const unsigned long long c1 = __builtin_amdgcn_s_memtime(), r1 = __builtin_amdgcn_s_memrealtime();
  if (threadIdx.x == 0) {
    clocks[2 * blockIdx.x] = c1 - c0;
    clocks[2 * blockIdx.x + 1] = r1 - r0;
  }
}

// ---- 4. The attention loop body, in the kernel's shape (H2 = 1) and with two heads per wave (H2 = 2).
__device__ __forceinline__ bf16x8 v_pair(const char* vt, const int* v_off, int k) {  // the V^T operand
  const char* a0 = vt + 16 * (k >> 2) * 256 + v_off[k & 3];
  const i16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) i16x4*)(a0));
  const i16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) i16x4*)(a0 + 2048));
  const i16x4 both[2] = {lo, hi};
  bf16x8 a;
  __builtin_memcpy(&a, both, sizeof(a));
  return a;
}

template <int H2>
__global__ void __launch_bounds__(512 / H2) loop_body(const char* src, float* sink, int iters,
                                                      unsigned long long* clocks) {
  const unsigned long long c0 = __builtin_amdgcn_s_memtime(), r0 = __builtin_amdgcn_s_memrealtime();
  constexpr int kWavesPerCu = 8 / H2;
  constexpr int kDma = 64 / kWavesPerCu;  // 1 KB DMA instructions per wave and iteration: 64 KB per CU
  __shared__ __attribute__((aligned(1024))) char k0[32768];
  __shared__ __attribute__((aligned(1024))) char k1[32768];
  __shared__ __attribute__((aligned(1024))) char v0[32768];
  __shared__ __attribute__((aligned(1024))) char v1[32768];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int part = H2 == 1 ? wave / 2 : wave;  // four KV parts, 8 KB tiles
  const int n = lane & 31;
  // the kernel's swizzled read offsets (K: chunk c of row r in slot c ^ (r % 16); V: c ^ 4 (r % 4))
  int k_off[8], v_off[4];
  for (int c = 0; c < 8; ++c) k_off[c] = part * 8192 + n * 256 + 16 * ((2 * c + (lane >> 5)) ^ (n & 15));
  const int tr_key = 4 * (lane >> 5) + ((lane & 15) >> 2);
  for (int m = 0; m < 4; ++m) {
    const int d = 32 * m + 16 * ((lane >> 4) & 1) + 4 * (lane & 3);
    v_off[m] = part * 8192 + tr_key * 256 + 16 * ((d >> 3) ^ ((tr_key & 3) << 2)) + 2 * (d & 7);
  }
  bf16x8 qreg[H2][8];
  for (int h = 0; h < H2; ++h)
    for (int c = 0; c < 8; ++c)
      for (int e = 0; e < 8; ++e) qreg[h][c][e] = (__bf16)((float)(((lane * 37 + h * 11 + c * 5 + e * 3) % 17) - 8) * 0.11f);
  f32x16 o_acc[H2][4], s_a[H2], s_b[H2];
  float m_run[H2], l_run[H2], m_tile[H2];
  for (int h = 0; h < H2; ++h) {
    for (int m = 0; m < 4; ++m) o_acc[h][m] = f32x16{};
    s_a[h] = f32x16{};
    s_b[h] = f32x16{};
    m_run[h] = l_run[h] = m_tile[h] = 0.0f;
  }
  const __amdgpu_buffer_rsrc_t rsrc = __builtin_amdgcn_make_buffer_rsrc((void*)src, (short)0, kSourceBytes, 0x00020000);
  const float c2 = 0.127f;
  // one iteration: state update, [QK^T of the next tile || exponentials of this tile, DMA into kw], then
  // [PV of this tile || last exponentials and the next tile's row max]
  auto iteration = [&](int it, f32x16* s_cur, f32x16* s_nxt, const char* kr, const char* vr, char* kw) {
    __builtin_amdgcn_s_waitcnt(0x0F70);
    __syncthreads();
    float shift[H2], rsum[H2], px[H2][16], tmax[H2];
    for (int h = 0; h < H2; ++h) {
      if (__any(m_tile[h] > m_run[h] + 8.0f)) {
        const float a = __builtin_amdgcn_exp2f(m_run[h] - m_tile[h]);
        l_run[h] *= a;
        for (int m = 0; m < 4; ++m) o_acc[h][m] *= a;
        m_run[h] = m_tile[h];
      }
      shift[h] = m_run[h];
      rsum[h] = 0.0f;
      tmax[h] = -INFINITY;
    }
    auto expo = [&](int h, int e) {
      px[h][e] = __builtin_amdgcn_exp2f(__builtin_fmaf(s_cur[h][e], c2, -shift[h]));
      rsum[h] += px[h][e];
    };
    bf16x8 kf[8], va[8];
    for (int k = 0; k < 3; ++k) kf[k] = *reinterpret_cast<const bf16x8*>(kr + k_off[k]);
    const unsigned src_base = (unsigned)((it * 64 + wave * kDma) % 1920) * 1024;  // < 2 MB - 64 KB
#pragma unroll
    for (int k = 0; k < 8; ++k) {
#pragma unroll
      for (int j = 0; j < kDma / 8; ++j) {
        const int i = k * (kDma / 8) + j;
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, LDS_PTR(kw + ((wave * kDma + i) % 32) * 1024), 16,
                                                 src_base + i * 1024 + lane * 16, 0, 0, 0);
      }
      if (k + 3 < 8) kf[k + 3] = *reinterpret_cast<const bf16x8*>(kr + k_off[k + 3]);
      else va[k - 5] = v_pair(vr, v_off, k - 5);
#pragma unroll
      for (int h = 0; h < H2; ++h)
        s_nxt[h] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kf[k], qreg[h][k], k == 0 ? f32x16{} : s_nxt[h], 0, 0, 0);
#pragma unroll
      for (int h = 0; h < H2; ++h) {
        expo(h, k);
        if ((k & 1) == 0) expo(h, 8 + (k >> 1));
      }
      __builtin_amdgcn_sched_barrier(0);
    }
    bf16x8 pb[H2][2];
    for (int h = 0; h < H2; ++h)
      for (int e = 0; e < 8; ++e) pb[h][0][e] = (__bf16)px[h][e];
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      if (k + 3 < 8) va[k + 3] = v_pair(vr, v_off, k + 3);
#pragma unroll
      for (int h = 0; h < H2; ++h) {
        if (k < 4) {
          expo(h, 12 + k);
          if (k == 3)
            for (int e = 8; e < 16; ++e) pb[h][1][e - 8] = (__bf16)px[h][e];
        }
        o_acc[h][k & 3] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(va[k], pb[h][k >> 2], o_acc[h][k & 3], 0, 0, 0);
        tmax[h] = fmaxf(fmaxf(tmax[h], s_nxt[h][2 * k]), s_nxt[h][2 * k + 1]);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
    for (int h = 0; h < H2; ++h) {
      l_run[h] += rsum[h];
      const unsigned u = __float_as_uint(tmax[h]);
      const auto r = __builtin_amdgcn_permlane32_swap(u, u, false, false);
      m_tile[h] = fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1])) * c2;
    }
  };
  for (int it = 0; it < iters; it += 2) {  // iters is even
    iteration(it, s_a, s_b, k1, v0, k0);
    iteration(it + 1, s_b, s_a, k0, v1, k1);
  }
  __builtin_amdgcn_s_waitcnt(0x0F70);
  float s = 0.0f;
  for (int h = 0; h < H2; ++h) {
    s += l_run[h] + m_run[h];
    for (int m = 0; m < 4; ++m)
      for (int e = 0; e < 16; ++e) s += o_acc[h][m][e];
  }
  sink[blockIdx.x * 512 + threadIdx.x] = s;
  const unsigned long long c1 = __builtin_amdgcn_s_memtime(), r1 = __builtin_amdgcn_s_memrealtime();
  if (threadIdx.x == 0) {
    clocks[2 * blockIdx.x] = c1 - c0;
    clocks[2 * blockIdx.x + 1] = r1 - r0;
  }
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

template <int H2>
void probe_loop_body(const char* src, float* sink, unsigned long long* clocks, const char* data) {
  const int iters = 1000;
  Timer t;
  float best = 1e30f;
  for (int r = 0; r < 3; ++r) {
    best = std::min(best, t.ms([&] { hipLaunchKernelGGL((loop_body<H2>), dim3(kCUs), dim3(512 / H2), 0, 0, src,
                                                        sink, iters, clocks); }));
  }
  unsigned long long h[2 * kCUs];
  CHECK(hipMemcpy(h, clocks, sizeof(h), hipMemcpyDeviceToHost));
  double cycles = 0, ticks100 = 0;
  for (int i = 0; i < kCUs; ++i) {
    cycles += double(h[2 * i]);
    ticks100 += double(h[2 * i + 1]);
  }
  std::printf("loop_body  %d head(s)/wave, %d waves/CU, K/V %-6s: %.3f us per iteration, shader clock %4.0f MHz, "
              "%4.0f cycles per iteration (MFMA alone: 1024)\n",
              H2, 8 / H2, data, best * 1e3 / iters, cycles / ticks100 * 100.0, cycles / kCUs / iters);
}

void probe_mfma_power(const char* src, float* sink, unsigned long long* clocks, int threads, const char* data) {
  const int rounds = 20000;
  Timer t;
  float last = 0.0f;
  for (int r = 0; r < 3; ++r) {  // the clock settles over the first launches: report the third
    last = t.ms([&] { hipLaunchKernelGGL(mfma_power, dim3(kCUs), dim3(threads), 0, 0,
                                         reinterpret_cast<const bf16x8*>(src), sink, rounds, clocks); });
  }
  unsigned long long h[2 * kCUs];
  CHECK(hipMemcpy(h, clocks, sizeof(h), hipMemcpyDeviceToHost));
  double cycles = 0, ticks100 = 0;
  for (int i = 0; i < kCUs; ++i) {
    cycles += double(h[2 * i]);
    ticks100 += double(h[2 * i + 1]);
  }
  const double mfma_per_simd = rounds * 8.0 * (threads / 256);
  const double tflops = mfma_per_simd * 4 * kCUs * 32768.0 / (last * 1e-3) / 1e12;
  std::printf("mfma_power waves/SIMD %d, operands %-6s: %6.2f ns per MFMA per SIMD, %6.0f TFLOP/s = %.2f of the "
              "bf16 peak, shader clock %4.0f MHz\n",
              threads / 256, data, last * 1e6 / mfma_per_simd, tflops, tflops / 2500.0, cycles / ticks100 * 100.0);
}

template <int kLdsBytes, int kThreads>
void probe_launch_floor(float* sink) {
  constexpr int kLaunches = 16, kReps = 50;
  hipStream_t s;
  CHECK(hipStreamCreate(&s));
  hipEvent_t a, b;
  CHECK(hipEventCreate(&a));
  CHECK(hipEventCreate(&b));
  auto step = [&] {
    for (int i = 0; i < kLaunches; ++i)
      hipLaunchKernelGGL((launch_floor<kLdsBytes, kThreads>), dim3(kCUs), dim3(kThreads), 0, s, sink);
  };
  auto per_launch_us = [&](auto run) {
    run();
    CHECK(hipStreamSynchronize(s));
    CHECK(hipEventRecord(a, s));
    for (int r = 0; r < kReps; ++r) run();
    CHECK(hipEventRecord(b, s));
    CHECK(hipEventSynchronize(b));
    float t = 0.0f;
    CHECK(hipEventElapsedTime(&t, a, b));
    return t * 1e3 / (kReps * kLaunches);
  };
  const float eager = per_launch_us([&] {
    step();
    CHECK(hipGetLastError());
  });
  hipGraph_t g;
  hipGraphExec_t ge;
  CHECK(hipStreamBeginCapture(s, hipStreamCaptureModeGlobal));
  step();
  CHECK(hipStreamEndCapture(s, &g));
  CHECK(hipGraphInstantiate(&ge, g, nullptr, nullptr, 0));
  const float graph = per_launch_us([&] { CHECK(hipGraphLaunch(ge, s)); });
  std::printf("launch_floor %3d threads/WG, %3d KB LDS, %d WGs: %5.2f us per launch back to back, %5.2f us per launch "
              "in a %d-launch HIP graph\n",
              kThreads, kLdsBytes / 1024, kCUs, eager, graph, kLaunches);
  CHECK(hipGraphExecDestroy(ge));
  CHECK(hipGraphDestroy(g));
  CHECK(hipEventDestroy(a));
  CHECK(hipEventDestroy(b));
  CHECK(hipStreamDestroy(s));
}

// Random bf16 values in [-1, 1) over the source buffer (a fixed LCG, so every run sees the same data).
void fill_random_bf16(char* src) {
  const size_t count = (kSourceBytes + 1024) / 2;
  unsigned short* host = static_cast<unsigned short*>(std::malloc(count * 2));
  unsigned x = 12345u;
  for (size_t i = 0; i < count; ++i) {
    x = x * 1664525u + 1013904223u;
    const float f = float((x >> 8) & 0xFFFF) / 32768.0f - 1.0f;
    unsigned u;
    std::memcpy(&u, &f, 4);
    host[i] = (unsigned short)(u >> 16);
  }
  CHECK(hipMemcpy(src, host, count * 2, hipMemcpyHostToDevice));
  std::free(host);
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
  unsigned long long* clocks = nullptr;
  CHECK(hipMalloc(&clocks, 2 * kCUs * sizeof(unsigned long long)));
  probe_loop_body<1>(src, sink, clocks, "zeros");
  probe_mfma_power(src, sink, clocks, 512, "zeros");
  fill_random_bf16(src);
  probe_loop_body<1>(src, sink, clocks, "random");
  probe_loop_body<2>(src, sink, clocks, "random");
  probe_mfma_power(src, sink, clocks, 512, "random");
  probe_mfma_power(src, sink, clocks, 256, "random");
  CHECK(hipFree(clocks));
  probe_launch_floor<147456, 512>(sink);
  probe_launch_floor<4096, 64>(sink);
  CHECK(hipFree(src));
  CHECK(hipFree(sink));
  CHECK(hipFree(ticks));
  return 0;
}
