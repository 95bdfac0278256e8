// Per-CU rates of the units the GEMMs and attention kernels lean on, measured on one MI355X:
// the MFMA pipe (v_mfma_f32_32x32x16_bf16), LDS reads (ds_read_b128), global -> LDS direct loads
// (global_load_lds_dwordx4) and global -> VGPR loads from an L2-resident buffer, and the mix of
// MFMA and LDS reads that a GEMM wave runs (with and without direct loads beside it), and the
// VALU issue of the softmax's exp2 against FMAs. Each line
// prints the wall time, the shader clock the kernel ran at (s_memtime against the 100 MHz
// s_memrealtime) and the rate. Build and run on the GPU host:
//   hipcc -O3 --offload-arch=gfx950 -Xclang -target-feature -Xclang -packed-fp32-ops \
//     sys1rust_amd/microbench/gfx950_rates.hip -o /tmp/gfx950_rates && /tmp/gfx950_rates
#include <hip/hip_runtime.h>

#include <cstdio>
#include <cstdlib>
#include <vector>

#define CK(x)                                                                          \
  do {                                                                                 \
    hipError_t e_ = (x);                                                               \
    if (e_ != hipSuccess) {                                                            \
      fprintf(stderr, "HIP %s at %s:%d\n", hipGetErrorString(e_), __FILE__, __LINE__); \
      exit(1);                                                                         \
    }                                                                                  \
  } while (0)

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

struct Clk {
  unsigned long long t0, t1, r0, r1;
};

__device__ void stamp(Clk* clk, unsigned long long t0, unsigned long long r0) {
  const unsigned long long t1 = __builtin_amdgcn_s_memtime(), r1 = __builtin_amdgcn_s_memrealtime();
  if (threadIdx.x == 0) clk[blockIdx.x] = {t0, t1, r0, r1};
}

// NACC independent MFMA chains per wave.
template <int NACC>
__global__ __launch_bounds__(256) void k_mfma(int iters, float* out, Clk* clk, const uint16_t*) {
  f32x16 acc[NACC];
  for (int i = 0; i < NACC; ++i)
    for (int e = 0; e < 16; ++e) acc[i][e] = 0;
  bf16x8 a, b;
  for (int e = 0; e < 8; ++e) {
    a[e] = (__bf16)(threadIdx.x * 0.001f);
    b[e] = (__bf16)(e * 0.01f);
  }
  const unsigned long long t0 = __builtin_amdgcn_s_memtime(), r0 = __builtin_amdgcn_s_memrealtime();
  for (int it = 0; it < iters; ++it)
#pragma unroll
    for (int i = 0; i < NACC; ++i) acc[i] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, acc[i], 0, 0, 0);
  stamp(clk, t0, r0);
  float s = 0;
  for (int i = 0; i < NACC; ++i)
    for (int e = 0; e < 16; ++e) s += acc[i][e];
  out[blockIdx.x * 256 + threadIdx.x] = s;
}

// NR conflict-free 16-byte LDS reads in flight per wave.
template <int NR>
__global__ __launch_bounds__(256) void k_lds(int iters, float* out, Clk* clk, const uint16_t*) {
  __shared__ __attribute__((aligned(16))) char sm[65536];
  for (int i = threadIdx.x; i < 65536 / 16; i += 256) reinterpret_cast<uint4*>(sm)[i] = make_uint4(i, i + 1, i + 2, i + 3);
  __syncthreads();
  uint4 x = make_uint4(0, 0, 0, 0);
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const unsigned long long t0 = __builtin_amdgcn_s_memtime(), r0 = __builtin_amdgcn_s_memrealtime();
  const int base = w * 16384 + lane * 16;
  for (int it = 0; it < iters; ++it) {
    uint4 v[NR];
#pragma unroll
    for (int r = 0; r < NR; ++r) v[r] = *reinterpret_cast<const uint4*>(sm + ((base + r * 1024 + it * 64) & 65535));
#pragma unroll
    for (int r = 0; r < NR; ++r) {
      x.x ^= v[r].x;
      x.y ^= v[r].y;
      x.z ^= v[r].z;
      x.w ^= v[r].w;
    }
  }
  stamp(clk, t0, r0);
  out[blockIdx.x * 256 + threadIdx.x] = float(x.x ^ x.y ^ x.z ^ x.w);
}

// Index of a 1 KiB block of the 1 MiB source: a wave's loads walk it, so most come from L2.
__device__ __forceinline__ size_t src_block(int l, int it) { return (size_t((blockIdx.x & 63) * 16 + l + it * 4) % 1024) * 512; }

// NL direct global -> LDS loads (1 KiB per wave each) per iteration, at most 8 in flight.
template <int NL>
__global__ __launch_bounds__(256) void k_gld(int iters, float* out, Clk* clk, const uint16_t* src) {
  __shared__ __attribute__((aligned(1024))) char sm[65536];
  const int lane = threadIdx.x & 63, w = __builtin_amdgcn_readfirstlane(int(threadIdx.x) >> 6);
  const unsigned long long t0 = __builtin_amdgcn_s_memtime(), r0 = __builtin_amdgcn_s_memrealtime();
  for (int it = 0; it < iters; ++it) {
#pragma unroll
    for (int l = 0; l < NL; ++l)
      __builtin_amdgcn_global_load_lds(src + src_block(l, it) + lane * 8, sm + (w * NL + l) % 64 * 1024, 16, 0, 0);
    asm volatile("s_waitcnt vmcnt(8)" ::: "memory");
  }
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
  stamp(clk, t0, r0);
  out[blockIdx.x * 256 + threadIdx.x] = float(sm[threadIdx.x * 4]);
}

// NL global -> VGPR 16-byte loads per iteration.
template <int NL>
__global__ __launch_bounds__(256) void k_gvr(int iters, float* out, Clk* clk, const uint16_t* src) {
  const int lane = threadIdx.x & 63;
  uint4 x = make_uint4(0, 0, 0, 0);
  const unsigned long long t0 = __builtin_amdgcn_s_memtime(), r0 = __builtin_amdgcn_s_memrealtime();
  for (int it = 0; it < iters; ++it) {
    uint4 v[NL];
#pragma unroll
    for (int l = 0; l < NL; ++l) v[l] = *reinterpret_cast<const uint4*>(src + src_block(l, it) + lane * 8);
#pragma unroll
    for (int l = 0; l < NL; ++l) {
      x.x ^= v[l].x;
      x.y += v[l].y;
    }
  }
  stamp(clk, t0, r0);
  out[blockIdx.x * 256 + threadIdx.x] = float(x.x ^ x.y);
}

// A GEMM wave's inner loop: FM x FN MFMAs per 16-k step on fragments read from LDS (FM + FN
// reads, double-buffered in registers), 4 steps per 64-k tile, plus NL direct loads per tile
// (issued over the first two steps, never awaited before the kernel's end; 0 = none).
template <int FM, int FN, int NL>
__global__ __launch_bounds__(256) void k_mix(int iters, float* out, Clk* clk, const uint16_t* src) {
  __shared__ __attribute__((aligned(1024))) char sm[81920];
  for (int i = threadIdx.x; i < 81920 / 16; i += 256) reinterpret_cast<uint4*>(sm)[i] = make_uint4(0x3c003c00u, i, 0, 0);
  __syncthreads();
  const int lane = threadIdx.x & 63, w = __builtin_amdgcn_readfirstlane(int(threadIdx.x) >> 6);
  constexpr int SPAN = NL ? 40960 : 81920;  // LDS the fragment reads use; direct loads write the rest
  f32x16 acc[FM][FN];
  for (int i = 0; i < FM; ++i)
    for (int j = 0; j < FN; ++j)
      for (int e = 0; e < 16; ++e) acc[i][j][e] = 0;
  const unsigned long long t0 = __builtin_amdgcn_s_memtime(), r0 = __builtin_amdgcn_s_memrealtime();
  bf16x8 af[2][FM], bw[2][FN];
  auto rd = [&](int ks, int buf) {
#pragma unroll
    for (int i = 0; i < FM; ++i)
      af[buf][i] = *reinterpret_cast<const bf16x8*>(sm + (((w * 8 + i) * 1024 + lane * 16 + ks * 4096) % SPAN));
#pragma unroll
    for (int j = 0; j < FN; ++j)
      bw[buf][j] = *reinterpret_cast<const bf16x8*>(sm + (((w * 8 + FM + j) * 1024 + lane * 16 + ks * 4096) % SPAN));
  };
  rd(0, 0);
  for (int it = 0; it < iters; ++it) {
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      if (NL && ks < 2) {
#pragma unroll
        for (int l = ks * (NL / 2); l < (ks + 1) * (NL / 2); ++l)
          __builtin_amdgcn_global_load_lds(src + src_block(l, it) + lane * 8, sm + 40960 + (w * NL + l) % 40 * 1024, 16, 0,
                                           0);
      }
      rd(it * 4 + ks + 1, (ks + 1) & 1);
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(bw[ks & 1][j], af[ks & 1][i], acc[i][j], 0, 0, 0);
    }
    if (NL) asm volatile("s_waitcnt vmcnt(20)" ::: "memory");
  }
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  stamp(clk, t0, r0);
  float s = 0;
  for (int i = 0; i < FM; ++i)
    for (int j = 0; j < FN; ++j)
      for (int e = 0; e < 16; ++e) s += acc[i][j][e];
  out[blockIdx.x * 256 + threadIdx.x] = s;
}

// VALU issue: 8 independent chains per lane of v_exp_f32 (MODE 0), v_fma_f32 (1), or half of
// each in every wave (2). Whether the transcendental overlaps the FMAs of the same wave shows in
// mode 2's time against the sum of the halves of modes 0 and 1.
template <int MODE>
__global__ __launch_bounds__(256) void k_valu(int iters, float* out, Clk* clk, const uint16_t*) {
  float x[8];
  for (int i = 0; i < 8; ++i) x[i] = threadIdx.x * 1e-4f - i * 0.01f;
  const unsigned long long t0 = __builtin_amdgcn_s_memtime(), r0 = __builtin_amdgcn_s_memrealtime();
  for (int it = 0; it < iters; ++it) {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const bool ex = MODE == 0 || (MODE == 2 && (i & 1) == 0);
      x[i] = ex ? __builtin_amdgcn_exp2f(x[i]) : fmaf(x[i], 0.999f, 1e-3f);
    }
  }
  stamp(clk, t0, r0);
  float s = 0;
  for (int i = 0; i < 8; ++i) s += x[i];
  out[blockIdx.x * 256 + threadIdx.x] = s;
}

template <class K>
void run(const char* name, K kern, int grid, int iters, double flop_per_wave_iter, double bytes_per_wave_iter,
         const uint16_t* src) {
  float* out;
  Clk* clk;
  CK(hipMalloc(&out, size_t(grid) * 256 * 4));
  CK(hipMalloc(&clk, grid * sizeof(Clk)));
  hipLaunchKernelGGL(kern, dim3(grid), dim3(256), 0, 0, iters, out, clk, src);  // warm-up
  CK(hipDeviceSynchronize());
  hipEvent_t a, b;
  CK(hipEventCreate(&a));
  CK(hipEventCreate(&b));
  CK(hipEventRecord(a, 0));
  hipLaunchKernelGGL(kern, dim3(grid), dim3(256), 0, 0, iters, out, clk, src);
  CK(hipEventRecord(b, 0));
  CK(hipEventSynchronize(b));
  float ms;
  CK(hipEventElapsedTime(&ms, a, b));
  std::vector<Clk> h(grid);
  CK(hipMemcpy(h.data(), clk, grid * sizeof(Clk), hipMemcpyDeviceToHost));
  double cyc = 0, rt = 0;
  for (const Clk& c : h) {
    cyc += double(c.t1 - c.t0);
    rt += double(c.r1 - c.r0);
  }
  const double ghz = cyc / (rt / 100e6) / 1e9;
  const double waves = grid * 4.0, sec = ms * 1e-3;
  const double tf = flop_per_wave_iter * waves * iters / sec / 1e12;
  const double bpc = bytes_per_wave_iter * waves * iters / sec / (ghz * 1e9) / 256.0;  // per CU per clock
  printf("%-34s %8.3f ms  %.2f GHz  %8.1f TFLOP/s  %6.1f B/clk/CU\n", name, ms, ghz, tf, bpc);
  CK(hipFree(out));
  CK(hipFree(clk));
}

int main() {
  const double mf = 32768.0;  // FLOPs of one 32x32x16 MFMA
  uint16_t* src;
  CK(hipMalloc(&src, 1024 * 512 * 2));  // 1 MiB, L2-resident
  CK(hipMemset(src, 0, 1024 * 512 * 2));
  run("mfma, 1 workgroup per CU", k_mfma<4>, 256, 20000, 4 * mf, 0, src);
  run("mfma, 2 workgroups per CU", k_mfma<4>, 512, 20000, 4 * mf, 0, src);
  run("lds read, 2 workgroups per CU", k_lds<8>, 512, 10000, 0, 8 * 1024, src);
  run("global->LDS, 2 workgroups per CU", k_gld<16>, 512, 2000, 0, 16 * 1024, src);
  run("global->VGPR, 2 workgroups per CU", k_gvr<8>, 512, 4000, 0, 8 * 1024, src);
  run("mfma+lds 96x64 wave, 2 per CU", k_mix<3, 2, 0>, 512, 2000, 4 * 6 * mf, 4 * 5 * 1024, src);
  run("  + 10 direct loads per k-tile", k_mix<3, 2, 10>, 512, 2000, 4 * 6 * mf, 4 * 5 * 1024, src);
  run("mfma+lds 96x64 wave, 16 k-tiles/WG", k_mix<3, 2, 0>, 1536, 16, 4 * 6 * mf, 4 * 5 * 1024, src);
  run("mfma+lds 128x128 wave, 1 per CU", k_mix<4, 4, 0>, 256, 2000, 4 * 16 * mf, 4 * 8 * 1024, src);
  run("mfma+lds 32x64 wave, 768 WGs", k_mix<1, 2, 0>, 768, 2000, 4 * 2 * mf, 4 * 3 * 1024, src);
  // The "TFLOP/s" column of these three is T lane-instructions/s (8 per lane per iteration).
  run("valu: exp2 only", k_valu<0>, 2048, 10000, 8 * 64, 0, src);
  run("valu: fma only", k_valu<1>, 2048, 10000, 8 * 64, 0, src);
  run("valu: half exp2, half fma per wave", k_valu<2>, 2048, 10000, 8 * 64, 0, src);
  CK(hipFree(src));
  return 0;
}
