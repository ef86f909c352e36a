// Backward of the gated residual that closes a DiT block's attention and FFN
// branches (x' = x + y·gate with a frozen gate; the forward is fused into the
// GEMM epilogue, gemm_kernel<C, true> in mlora_gemm.hip):
//
//   mlora_gate_scale_rows : dY[m, n] = bf16(dX'[m, n] · gate[m / gate_rows, n])
//
// one fp32 multiply rounded to nearest, as the reference's frozen-gate
// backward (runtime/helios_residual_kernel.py:90-133); the gradient of x is dX'
// itself. One wave per row, 16-byte loads and stores: 2 + 4 / gate_rows bytes
// read and 2 written per element, HBM-bound.
#include "mlora_common.h"
#include "mlora_host.h"

namespace mlora {

struct GateScaleArgs {
  const uint16_t *dout;
  const float *gate;
  uint16_t *dy;
  int64_t ldout, ldgate, lddy;
  int32_t M, N, gate_rows;
};

__global__ __launch_bounds__(256) void gate_scale_kernel(const GateScaleArgs a) {
  const int lane = threadIdx.x & 63;
  const int m = blockIdx.x * 4 + wave_id();
  if (m >= a.M) return;
  const uint16_t *orow = a.dout + (int64_t)m * a.ldout;
  const float *grow = a.gate + (int64_t)(m / a.gate_rows) * a.ldgate;
  uint16_t *yrow = a.dy + (int64_t)m * a.lddy;
  for (int n = 8 * lane; n < a.N; n += 512) {
    const u32x4 v = *(const MLORA_GLOBAL u32x4 *)(orow + n);
    const f32x4 g0 = *(const MLORA_GLOBAL f32x4 *)(grow + n), g1 = *(const MLORA_GLOBAL f32x4 *)(grow + n + 4);
    uint32_t o[4];
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      const float ga = w < 2 ? g0[2 * w] : g1[2 * w - 4], gb = w < 2 ? g0[2 * w + 1] : g1[2 * w - 3];
      o[w] = pack2_bf16(bf16_to_f32(v[w] & 0xffff) * ga, bf16_to_f32(v[w] >> 16) * gb);
    }
    *(MLORA_GLOBAL u32x4 *)(yrow + n) = u32x4{o[0], o[1], o[2], o[3]};
  }
}

}  // namespace mlora

using namespace mlora;

extern "C" int mlora_gate_scale_rows(const void *dout, int64_t ldout, int64_t M, int64_t N, const float *gate,
                                     int64_t ldgate, int64_t gate_rows, void *dy, int64_t lddy, void *stream) {
  if (M < 0 || N < 0) return MLORA_ERR_INVALID;
  if (M > INT32_MAX - 4 || N > INT32_MAX / 2) return MLORA_ERR_LIMIT;
  int st = check_bf16_matrix(dout, ldout, M, N);
  if (st) return st;
  if ((st = check_bf16_matrix(dy, lddy, M, N))) return st;
  if (M == 0 || N == 0) return MLORA_OK;
  if (gate == nullptr || gate_rows < 1 || gate_rows > INT32_MAX) return MLORA_ERR_INVALID;
  if (ldgate < N || ldgate % 4 != 0 || !aligned16(gate)) return MLORA_ERR_UNSUPPORTED;
  GateScaleArgs a{static_cast<const uint16_t *>(dout), gate, static_cast<uint16_t *>(dy), ldout, ldgate, lddy,
                  (int32_t)M, (int32_t)N, (int32_t)gate_rows};
  hipLaunchKernelGGL(gate_scale_kernel, dim3((unsigned)((M + 3) / 4)), dim3(256), 0, static_cast<hipStream_t>(stream),
                     a);
  return launch_status();
}
