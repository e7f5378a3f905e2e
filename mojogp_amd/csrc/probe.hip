// Instruction-throughput probe of the gfx950 pipes the tile kernel uses:
// transcendental VALU (v_exp_f32), plain VALU (v_fma_f32), 16-bit K=32 MFMA
// (v_mfma_f32_16x16x32_f16), and the MFMA cost when interleaved with VALU work
// of the same waves (4 MFMA + 16 FMA per iteration).  Each probe runs 2048
// workgroups of 256 threads (8 waves per SIMD) through kIters iterations of
// independent chains; the shader clock comes from s_memtime against the
// 100 MHz s_memrealtime counter read by one wave.  Results are cycles per
// wave-instruction per SIMD, the unit of the tile kernel's pipe model.
#include <cstdint>

#include "mojogp_amd.h"
#include "mgp_common.h"

namespace mgp {
namespace {

typedef float f4 __attribute__((ext_vector_type(4)));
typedef _Float16 h8 __attribute__((ext_vector_type(8)));

constexpr int kIters = 2048;
constexpr int kProbeBlocks = 2048, kProbeThreads = 256;

// Clock sample of workgroup 7, wave 0: [shader cycles, 100 MHz ticks].
__global__ void k_probe_trans(float* out, unsigned long long* clk) {
  float x[8];
  for (int k = 0; k < 8; ++k) x[k] = 1e-3f * (threadIdx.x + k);
  const unsigned long long c0 = __builtin_amdgcn_s_memtime(), r0 = __builtin_amdgcn_s_memrealtime();
  for (int it = 0; it < kIters; ++it) {
#pragma unroll
    for (int k = 0; k < 8; ++k) x[k] = __builtin_amdgcn_exp2f(-x[k]);
  }
  const unsigned long long c1 = __builtin_amdgcn_s_memtime(), r1 = __builtin_amdgcn_s_memrealtime();
  float s = 0.f;
  for (int k = 0; k < 8; ++k) s += x[k];
  out[blockIdx.x * blockDim.x + threadIdx.x] = s;
  if (blockIdx.x == 7 && threadIdx.x == 0) {
    clk[0] = c1 - c0;
    clk[1] = r1 - r0;
  }
}

__global__ void k_probe_valu(float* out, float a, float b) {
  float x[8];
  for (int k = 0; k < 8; ++k) x[k] = 1e-3f * (threadIdx.x + k);
  for (int it = 0; it < kIters; ++it) {
#pragma unroll
    for (int k = 0; k < 8; ++k) x[k] = fmaf(x[k], a, b);
  }
  float s = 0.f;
  for (int k = 0; k < 8; ++k) s += x[k];
  out[blockIdx.x * blockDim.x + threadIdx.x] = s;
}

__device__ __forceinline__ void probe_operands(h8& a, h8& b) {
  for (int k = 0; k < 8; ++k) {
    a[k] = (_Float16)(1e-3f * (threadIdx.x & 63));
    b[k] = (_Float16)2e-3f;
  }
}

__global__ void k_probe_mfma(float* out) {
  f4 acc[4];
  for (int k = 0; k < 4; ++k) acc[k] = f4{0.f, 0.f, 0.f, 0.f};
  h8 a, b;
  probe_operands(a, b);
  for (int it = 0; it < kIters; ++it) {
#pragma unroll
    for (int k = 0; k < 4; ++k) acc[k] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, acc[k], 0, 0, 0);
  }
  float s = 0.f;
  for (int k = 0; k < 4; ++k) s += acc[k][0] + acc[k][1] + acc[k][2] + acc[k][3];
  out[blockIdx.x * blockDim.x + threadIdx.x] = s;
}

__global__ void k_probe_mix(float* out, float a2, float b2) {
  f4 acc[4];
  for (int k = 0; k < 4; ++k) acc[k] = f4{0.f, 0.f, 0.f, 0.f};
  h8 a, b;
  probe_operands(a, b);
  float x[8];
  for (int k = 0; k < 8; ++k) x[k] = 1e-3f * (threadIdx.x + k);
  for (int it = 0; it < kIters; ++it) {
#pragma unroll
    for (int k = 0; k < 4; ++k) acc[k] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, acc[k], 0, 0, 0);
#pragma unroll
    for (int k = 0; k < 8; ++k) x[k] = fmaf(x[k], a2, b2);
#pragma unroll
    for (int k = 0; k < 8; ++k) x[k] = fmaf(x[k], a2, b2);
  }
  float s = 0.f;
  for (int k = 0; k < 4; ++k) s += acc[k][0] + acc[k][1] + acc[k][2] + acc[k][3];
  for (int k = 0; k < 8; ++k) s += x[k];
  out[blockIdx.x * blockDim.x + threadIdx.x] = s;
}

}  // namespace
}  // namespace mgp

using namespace mgp;

extern "C" int mgp_pipe_probe(double* out, int nout) {
  return guarded([&] {
    MGP_REQUIRE(out != nullptr && nout >= 6, "mgp_pipe_probe needs an output array of 6 doubles");
    int dev = 0, cus = 0;
    MGP_HIP_CHECK(hipGetDevice(&dev));
    MGP_HIP_CHECK(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev));
    DevBuf<float> sink;
    sink.ensure((size_t)kProbeBlocks * kProbeThreads);
    DevBuf<unsigned long long> clk;
    clk.ensure(2);
    hipEvent_t e0, e1;
    MGP_HIP_CHECK(hipEventCreate(&e0));
    MGP_HIP_CHECK(hipEventCreate(&e1));
    const double waves = (double)kProbeBlocks * kProbeThreads / 64.0;
    const double simds = 4.0 * cus;
    // ms per launch: the average of 5 launches after one warm-up
    auto time = [&](auto launch) -> double {
      launch();
      MGP_HIP_CHECK(hipGetLastError());
      MGP_HIP_CHECK(hipDeviceSynchronize());
      MGP_HIP_CHECK(hipEventRecord(e0, 0));
      for (int r = 0; r < 5; ++r) launch();
      MGP_HIP_CHECK(hipEventRecord(e1, 0));
      MGP_HIP_CHECK(hipEventSynchronize(e1));
      float ms = 0.f;
      MGP_HIP_CHECK(hipEventElapsedTime(&ms, e0, e1));
      return ms / 5.0;
    };
    const dim3 g(kProbeBlocks), b(kProbeThreads);
    const double ms_trans = time([&] { hipLaunchKernelGGL(k_probe_trans, g, b, 0, 0, sink.ptr, clk.ptr); });
    unsigned long long cyc[2] = {0, 0};
    MGP_HIP_CHECK(hipMemcpy(cyc, clk.ptr, sizeof cyc, hipMemcpyDeviceToHost));
    const double ghz = cyc[1] > 0 ? (double)cyc[0] / ((double)cyc[1] * 10.0) : 0.0;
    const double ms_valu = time([&] { hipLaunchKernelGGL(k_probe_valu, g, b, 0, 0, sink.ptr, 0.5f, 0.25f); });
    const double ms_mfma = time([&] { hipLaunchKernelGGL(k_probe_mfma, g, b, 0, 0, sink.ptr); });
    const double ms_mix = time([&] { hipLaunchKernelGGL(k_probe_mix, g, b, 0, 0, sink.ptr, 0.5f, 0.25f); });
    (void)hipEventDestroy(e0);
    (void)hipEventDestroy(e1);
    // cycles per wave-instruction per SIMD = ms * 1e6 ns * GHz / (wave-instructions / SIMD)
    auto cyc_per = [&](double ms, double instr_per_iter) {
      return ms * 1e6 * ghz / (waves * kIters * instr_per_iter / simds);
    };
    out[0] = ghz;
    out[1] = cyc_per(ms_trans, 8);
    out[2] = cyc_per(ms_valu, 8);
    out[3] = cyc_per(ms_mfma, 4);
    // MFMA cost inside a VALU stream: (mixed iteration - its 16 FMAs) / 4
    out[4] = (cyc_per(ms_mix, 20) * 20.0 - 16.0 * out[2]) / 4.0;
    out[5] = (double)cus;
  });
}
