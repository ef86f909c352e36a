// Backward of the gated residual that closes a DiT block's attention and FFN
// branches (x' = x + y·gate with a frozen gate; the forward is fused into the
// GEMM epilogue, gemm_kernel<C, true> in mlora_gemm.hip):
//
//   mlora_gate_scale_rows : dY[m, n] = bf16(dX'[m, n] · gate[m / gate_rows, n])
//
// one fp32 multiply rounded to nearest, as the reference's frozen-gate
// backward (runtime/helios_residual_kernel.py:90-133); the gradient of x is dX'
// itself. dX' is bf16 (bf16 residual stream) or float32 (the Wan block's float32
// stream, reference/livewan_wan21/wan/modules/model.py:305-306: the bf16 y enters
// x + y·e as float32, so autograd hands y bf16(dX'·e)). One wave per row, 16-byte
// loads and stores, HBM-bound.
#include "mlora_common.h"
#include "mlora_host.h"

namespace mlora {

struct GateScaleArgs {
  const void *dout;  // bf16, or float32 when dout_f32
  const float *gate;
  uint16_t *dy;
  int64_t ldout, ldgate, lddy;
  int32_t M, N, gate_rows;
  int32_t dout_f32;
};

__global__ __launch_bounds__(256) void gate_scale_kernel(const GateScaleArgs a) {
  const int lane = threadIdx.x & 63;
  const int m = blockIdx.x * 4 + wave_id();
  if (m >= a.M) return;
  const float *grow = a.gate + (int64_t)(m / a.gate_rows) * a.ldgate;
  uint16_t *yrow = a.dy + (int64_t)m * a.lddy;
  for (int n = 8 * lane; n < a.N; n += 512) {
    float v[8];
    if (a.dout_f32) {
      const float *orow = static_cast<const float *>(a.dout) + (int64_t)m * a.ldout;
      const f32x4 v0 = *(const MLORA_GLOBAL f32x4 *)(orow + n), v1 = *(const MLORA_GLOBAL f32x4 *)(orow + n + 4);
#pragma unroll
      for (int e = 0; e < 4; ++e) v[e] = v0[e], v[e + 4] = v1[e];
    } else {
      const uint16_t *orow = static_cast<const uint16_t *>(a.dout) + (int64_t)m * a.ldout;
      const u32x4 u = *(const MLORA_GLOBAL u32x4 *)(orow + n);
#pragma unroll
      for (int e = 0; e < 8; ++e) v[e] = bf16_to_f32((uint16_t)(e % 2 ? u[e / 2] >> 16 : u[e / 2] & 0xffff));
    }
    const f32x4 g0 = *(const MLORA_GLOBAL f32x4 *)(grow + n), g1 = *(const MLORA_GLOBAL f32x4 *)(grow + n + 4);
    uint32_t o[4];
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      const float ga = w < 2 ? g0[2 * w] : g1[2 * w - 4], gb = w < 2 ? g0[2 * w + 1] : g1[2 * w - 3];
      o[w] = pack2_bf16(v[2 * w] * ga, v[2 * w + 1] * gb);
    }
    *(MLORA_GLOBAL u32x4 *)(yrow + n) = u32x4{o[0], o[1], o[2], o[3]};
  }
}

}  // namespace mlora

using namespace mlora;

extern "C" int mlora_gate_scale_rows(const void *dout, int64_t ldout, int64_t M, int64_t N, const float *gate,
                                     int64_t ldgate, int64_t gate_rows, void *dy, int64_t lddy, int dout_dtype,
                                     void *stream) {
  if (M < 0 || N < 0) return MLORA_ERR_INVALID;
  if (M > INT32_MAX - 4 || N > INT32_MAX / 2) return MLORA_ERR_LIMIT;
  if (dout_dtype != MLORA_BF16 && dout_dtype != MLORA_F32) return MLORA_ERR_UNSUPPORTED;
  int st = MLORA_OK;
  if (dout_dtype == MLORA_BF16) {
    st = check_bf16_matrix(dout, ldout, M, N);
  } else if (M > 0 && N > 0) {  // float32 rows of 16-byte chunks
    if (dout == nullptr || ldout < N) st = MLORA_ERR_INVALID;
    else if (!aligned16(dout) || ldout % 4 != 0 || N % 8 != 0) st = MLORA_ERR_UNSUPPORTED;
  }
  if (st) return st;
  if ((st = check_bf16_matrix(dy, lddy, M, N))) return st;
  if (M == 0 || N == 0) return MLORA_OK;
  if (gate == nullptr || gate_rows < 1 || gate_rows > INT32_MAX) return MLORA_ERR_INVALID;
  if (ldgate < N || ldgate % 4 != 0 || !aligned16(gate)) return MLORA_ERR_UNSUPPORTED;
  GateScaleArgs a{dout, gate, static_cast<uint16_t *>(dy), ldout, ldgate, lddy,
                  (int32_t)M, (int32_t)N, (int32_t)gate_rows, dout_dtype == MLORA_F32 ? 1 : 0};
  hipLaunchKernelGGL(gate_scale_kernel, dim3((unsigned)((M + 3) / 4)), dim3(256), 0, static_cast<hipStream_t>(stream),
                     a);
  return launch_status();
}
