// fp32 arithmetic path of the multi-LoRA linear: every operand, product and sum in
// IEEE float32 on the gfx950 fp32 matrix core (v_mfma_f32_32x32x2_f32).
//
// This is the reference's `precision='fp32'` mode: the native model runs without
// autocast (training/single_device.py:77-80), so TrainableLowRankLinear sees fp32
// x, W, lora_a, lora_b and computes base(x) + s·F.linear(F.linear(x, A), B) in fp32
// (training/low_rank.py:26-28), and autograd's backward in fp32.
//
//   shrink      h[m, j]  = s_a · Σ_k P[m,k]·Op_a(j,k)          (X·Aᵀ, s·dY·B)
//   gemm_fwd    Y[m, n]  = Σ_k X[m,k]·W[n,k] + b[n] + Σ_j h[m,j]·B_a[n,j]
//   gemm_dx     dX[m, k] = Σ_n dY[m,n]·W[n,k] + Σ_j g[m,j]·A_a[j,k]
//   seg_outer   D_a[c, j] = Σ_{m ∈ rows of a} P[m,c]·H[m,j]      (dB_a, dA_aᵀ)
//
// One tile kernel serves all four: a 128 x 128 output tile, 4 waves of 64 x 64
// (2 x 2 MFMA tiles of 32 x 32), contraction in k-tiles of 16 through two LDS
// buffers (the next k-tile is loaded into registers while the current one is
// multiplied). Each operand is a logical matrix O(r, k) = base[r·sr + k·sk] whose
// rows outside [r_lo, r_hi) and contraction indices >= klen read as zero; a tile
// sums a fixed, ordered list of such (P, Q) sources, so the result is
// deterministic and the LoRA term is more contraction in the same accumulators.
// LDS holds both operands k-major ([k][r]), so an MFMA fragment read (lane l:
// row l % 32 of k-row l / 32) is two runs of 32 consecutive floats.
#include "mlora_common.h"
#include "mlora_host.h"

namespace mlora {

constexpr int FB = 128;      // output tile rows and columns
constexpr int FK = 16;       // contraction per k-tile
constexpr int FLD = FB + 4;  // floats per LDS k-row

// O(r, k) = base[r·sr + k·sk] for r in [r_lo, r_hi), k < klen; zero elsewhere.
struct F32Op {
  const float *base;
  int64_t sr, sk;
  int32_t r_lo, r_hi, klen;
};

// A 128 x 16 tile of an operand, 8 values per thread. CK: the operand is
// contiguous along k (4 consecutive k per thread), else along r (4 consecutive r).
template <bool CK>
struct F32Tile {
  float v[8];
  __device__ __forceinline__ static void coords(int e, int tid, int &rl, int &kl) {
    if constexpr (CK) {
      rl = (tid >> 2) + 64 * (e >> 2);
      kl = 4 * (tid & 3) + (e & 3);
    } else {
      kl = (tid >> 5) + 8 * (e >> 2);
      rl = 4 * (tid & 31) + (e & 3);
    }
  }
  __device__ __forceinline__ void load(const F32Op &o, int r0, int k0, int tid) {
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      int rl, kl;
      coords(e, tid, rl, kl);
      const int r = r0 + rl, k = k0 + kl;
      const bool ok = r >= o.r_lo && r < o.r_hi && k < o.klen;
      v[e] = ok ? o.base[(int64_t)r * o.sr + (int64_t)k * o.sk] : 0.f;
    }
  }
  __device__ __forceinline__ void store(float *lds, int tid) const {
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      int rl, kl;
      coords(e, tid, rl, kl);
      lds[kl * FLD + rl] = v[e];
    }
  }
};

// One k-tile: wave (wi, wj) multiplies rows 64wi.. of P by columns 64wj.. of Q.
// MFMA 32x32x2: lane l gives A[row l % 32][k l / 32] and B[k l / 32][col l % 32];
// acc register v of lane l is C[8(v / 4) + 4(l / 32) + v % 4][l % 32].
__device__ __forceinline__ void f32_mma(f32x16 (&acc)[2][2], const float *lp, const float *lq, int wi, int wj,
                                        int lane, float scale) {
#pragma unroll
  for (int kk = 0; kk < FK; kk += 2) {
    const int kr = (kk + (lane >> 5)) * FLD + (lane & 31);
    float a[2], b[2];
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      a[t] = lp[kr + 64 * wi + 32 * t] * scale;
      b[t] = lq[kr + 64 * wj + 32 * t];
    }
#pragma unroll
    for (int ti = 0; ti < 2; ++ti)
#pragma unroll
      for (int tj = 0; tj < 2; ++tj)
        acc[ti][tj] = __builtin_amdgcn_mfma_f32_32x32x2f32(a[ti], b[tj], acc[ti][tj], 0, 0, 0);
  }
}

// acc += scale · Σ_k P(i0 + ·, k)·Q(j0 + ·, k) over the whole contraction of one
// source. Two LDS buffers; every wave passes the same barriers.
template <bool PCK, bool QCK>
__device__ __forceinline__ void f32_contract(f32x16 (&acc)[2][2], const F32Op &p, const F32Op &q, float scale, int i0,
                                             int j0, float *lds, int tid, int wi, int wj, int lane) {
  const int nk = (p.klen + FK - 1) / FK;
  if (nk <= 0) return;
  float *bp[2] = {lds, lds + 2 * FK * FLD};
  float *bq[2] = {lds + FK * FLD, lds + 3 * FK * FLD};
  F32Tile<PCK> tp;
  F32Tile<QCK> tq;
  tp.load(p, i0, 0, tid);
  tq.load(q, j0, 0, tid);
  __syncthreads();  // the previous source's last k-tile has been read by every wave
  tp.store(bp[0], tid);
  tq.store(bq[0], tid);
  __syncthreads();
  for (int kt = 0; kt < nk; ++kt) {
    const int cur = kt & 1;
    const bool more = kt + 1 < nk;
    if (more) {
      tp.load(p, i0, (kt + 1) * FK, tid);
      tq.load(q, j0, (kt + 1) * FK, tid);
    }
    f32_mma(acc, bp[cur], bq[cur], wi, wj, lane, scale);
    if (more) {
      tp.store(bp[cur ^ 1], tid);
      tq.store(bq[cur ^ 1], tid);
    }
    __syncthreads();
  }
}

// ---------------------------------------------------------------- linear / shrink

struct F32LinArgs {
  const float *P;  // [M, Kc] row-major (pitch ldp)
  int64_t ldp;
  const float *Q;  // main operand: Q(j, k) = Q[j·q_sr + k·q_sk]
  int64_t q_sr, q_sk;
  const float *E;  // LoRA rows [M, >= r] (pitch lde) of the fused GEMMs
  int64_t lde;
  const float *bias;
  float *C;
  int64_t ldc;
  int32_t M, Ncols, Kc;
  int32_t tiles_n;
  int32_t shrink;  // 1: no main term; the sources are P·Op_a over Kc, scaled by s_a
  const float *qe[kMaxAdapters];
  int64_t qe_sr[kMaxAdapters], qe_sk[kMaxAdapters];
  int32_t rank[kMaxAdapters];
  float scale[kMaxAdapters];
  SegTable seg;
};

template <bool QCK>
__global__ __launch_bounds__(256) void f32_linear_kernel(const F32LinArgs a) {
  __shared__ float lds[4 * FK * FLD];
  const int tid = threadIdx.x, lane = tid & 63, wave = wave_id();
  const int wi = wave >> 1, wj = wave & 1;
  const int i0 = (blockIdx.x / a.tiles_n) * FB, j0 = (blockIdx.x % a.tiles_n) * FB;
  f32x16 acc[2][2];
#pragma unroll
  for (int ti = 0; ti < 2; ++ti)
#pragma unroll
    for (int tj = 0; tj < 2; ++tj)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[ti][tj][v] = 0.f;
  if (!a.shrink && a.Kc > 0) {
    const F32Op p{a.P, a.ldp, 1, 0, a.M, a.Kc};
    const F32Op q{a.Q, a.q_sr, a.q_sk, 0, a.Ncols, a.Kc};
    f32_contract<true, QCK>(acc, p, q, 1.f, i0, j0, lds, tid, wi, wj, lane);
  }
  const int iend = min(i0 + FB, a.M);
  for (int s = seg_of_row(a.seg, i0); s < a.seg.n && a.seg.off[s] < iend; ++s) {
    const int ad = a.seg.aid[s];
    if (ad < 0 || a.rank[ad] == 0 || a.seg.off[s + 1] <= i0 || a.seg.off[s + 1] == a.seg.off[s]) continue;
    const int r = a.rank[ad];
    if (a.shrink) {
      const F32Op p{a.P, a.ldp, 1, a.seg.off[s], a.seg.off[s + 1], a.Kc};
      const F32Op q{a.qe[ad], a.qe_sr[ad], a.qe_sk[ad], 0, r, a.Kc};
      f32_contract<true, QCK>(acc, p, q, a.scale[ad], i0, j0, lds, tid, wi, wj, lane);
    } else {
      const F32Op p{a.E, a.lde, 1, a.seg.off[s], a.seg.off[s + 1], r};
      const F32Op q{a.qe[ad], a.qe_sr[ad], a.qe_sk[ad], 0, a.Ncols, r};
      f32_contract<true, QCK>(acc, p, q, 1.f, i0, j0, lds, tid, wi, wj, lane);
    }
  }
#pragma unroll
  for (int ti = 0; ti < 2; ++ti)
#pragma unroll
    for (int tj = 0; tj < 2; ++tj) {
      const int j = j0 + 64 * wj + 32 * tj + (lane & 31);
      if (j >= a.Ncols) continue;
      const float b = a.bias ? a.bias[j] : 0.f;
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int i = i0 + 64 * wi + 32 * ti + 8 * (v >> 2) + 4 * (lane >> 5) + (v & 3);
        if (i < a.M) a.C[(int64_t)i * a.ldc + j] = acc[ti][tj][v] + b;
      }
    }
}

// ---------------------------------------------------------------- segmented outer product

struct F32OuterArgs {
  const float *P;  // [M, Ci] (pitch ldp): P(i, k = m) = P[m·ldp + i]
  int64_t ldp;
  const float *H;  // [M, >= r] (pitch ldh): Q(j, k = m) = H[m·ldh + j]
  int64_t ldh;
  int32_t Ci;
  int32_t tiles_j;
  int32_t out_layout;  // 0: D_a [Ci, r_a]; 1: D_a [r_a, Ci]
  float *out[kMaxAdapters];
  int32_t rank[kMaxAdapters];
  SegTable seg;
};

// Grid (tiles of [Ci, max r], adapters): adapter a's segments in routing order.
__global__ __launch_bounds__(256) void f32_outer_kernel(const F32OuterArgs a) {
  __shared__ float lds[4 * FK * FLD];
  const int ad = blockIdx.y;
  const int r = a.rank[ad];
  if (r == 0 || a.out[ad] == nullptr) return;  // the whole workgroup
  const int i0 = (blockIdx.x / a.tiles_j) * FB, j0 = (blockIdx.x % a.tiles_j) * FB;
  if (j0 >= r) return;
  const int tid = threadIdx.x, lane = tid & 63, wave = wave_id();
  const int wi = wave >> 1, wj = wave & 1;
  f32x16 acc[2][2];
#pragma unroll
  for (int ti = 0; ti < 2; ++ti)
#pragma unroll
    for (int tj = 0; tj < 2; ++tj)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[ti][tj][v] = 0.f;
  for (int s = 0; s < a.seg.n; ++s) {
    const int lo = a.seg.off[s], len = a.seg.off[s + 1] - lo;
    if (a.seg.aid[s] != ad || len == 0) continue;
    const F32Op p{a.P + (int64_t)lo * a.ldp, 1, a.ldp, 0, a.Ci, len};
    const F32Op q{a.H + (int64_t)lo * a.ldh, 1, a.ldh, 0, r, len};
    f32_contract<false, false>(acc, p, q, 1.f, i0, j0, lds, tid, wi, wj, lane);
  }
  float *o = a.out[ad];
#pragma unroll
  for (int ti = 0; ti < 2; ++ti)
#pragma unroll
    for (int tj = 0; tj < 2; ++tj) {
      const int j = j0 + 64 * wj + 32 * tj + (lane & 31);
      if (j >= r) continue;
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int i = i0 + 64 * wi + 32 * ti + 8 * (v >> 2) + 4 * (lane >> 5) + (v & 3);
        if (i >= a.Ci) continue;
        o[a.out_layout == 0 ? (int64_t)i * r + j : (int64_t)j * a.Ci + i] = acc[ti][tj][v];
      }
    }
}

// ---------------------------------------------------------------- host side

static bool aligned4(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 3u) == 0; }

// fp32 row-major matrix [rows, cols], pitch ld (elements).
static int check_f32_matrix(const void *p, int64_t ld, int64_t rows, int64_t cols) {
  if (rows == 0 || cols == 0) return MLORA_OK;
  if (p == nullptr || ld < cols) return MLORA_ERR_INVALID;
  if (!aligned4(p)) return MLORA_ERR_UNSUPPORTED;
  return MLORA_OK;
}

// Adapter operands for the fp32 kernels: any rank in [0, kMaxRank] (no padding).
static int f32_adapters(F32LinArgs &a, const void *const *ptrs, const int32_t *ranks, const float *scales, int32_t n) {
  if (n < 0) return MLORA_ERR_INVALID;
  if (n > kMaxAdapters) return MLORA_ERR_LIMIT;
  if (n > 0 && ranks == nullptr) return MLORA_ERR_INVALID;
  for (int i = 0; i < kMaxAdapters; ++i) {
    a.qe[i] = nullptr;
    a.rank[i] = 0;
    a.scale[i] = 0.f;
    a.qe_sr[i] = a.qe_sk[i] = 0;
  }
  for (int i = 0; i < n; ++i) {
    if (ranks[i] < 0) return MLORA_ERR_INVALID;
    if (ranks[i] > kMaxRank) return MLORA_ERR_LIMIT;
    a.rank[i] = ranks[i];
    a.scale[i] = scales ? scales[i] : 1.f;
    if (ranks[i] > 0 && adapter_used(a.seg, i)) {
      if (ptrs == nullptr || ptrs[i] == nullptr) return MLORA_ERR_INVALID;
      if (!aligned4(ptrs[i])) return MLORA_ERR_UNSUPPORTED;
      a.qe[i] = static_cast<const float *>(ptrs[i]);
    }
  }
  return MLORA_OK;
}

static int f32_max_rank(const F32LinArgs &a) {
  int r = 0;
  for (int s = 0; s < a.seg.n; ++s) {
    const int ad = a.seg.aid[s];
    if (ad >= 0 && a.seg.off[s + 1] > a.seg.off[s] && a.rank[ad] > r) r = a.rank[ad];
  }
  return r;
}

static int f32_launch_linear(F32LinArgs &a, bool qck, hipStream_t stream) {
  const int64_t tm = (a.M + FB - 1) / FB, tn = (a.Ncols + FB - 1) / FB;
  if (tm == 0 || tn == 0) return MLORA_OK;
  if (tm * tn > INT32_MAX) return MLORA_ERR_LIMIT;
  a.tiles_n = (int32_t)tn;
  if (qck)
    hipLaunchKernelGGL(f32_linear_kernel<true>, dim3((unsigned)(tm * tn)), dim3(256), 0, stream, a);
  else
    hipLaunchKernelGGL(f32_linear_kernel<false>, dim3((unsigned)(tm * tn)), dim3(256), 0, stream, a);
  return launch_status();
}

static bool f32_dims_ok(int64_t M, int64_t K, int64_t N) {
  return M >= 0 && K >= 0 && N >= 0 && M <= INT32_MAX - FB && K <= INT32_MAX - FB && N <= INT32_MAX - FB;
}

}  // namespace mlora

using namespace mlora;

extern "C" int mlora_f32_shrink(const void *p, int64_t ldp, int64_t M, int64_t K, const void *const *op_ptrs,
                                int op_layout, const int32_t *ranks, const float *scales, int32_t n_adapters,
                                const int64_t *seg_offsets, const int32_t *adapter_ids, int32_t n_segments, void *h,
                                int64_t ldh, int64_t width, void *stream) {
  F32LinArgs a{};
  if (!f32_dims_ok(M, K, width)) return MLORA_ERR_LIMIT;
  int st = build_segtable(a.seg, M, seg_offsets, adapter_ids, n_segments, n_adapters);
  if (st) return st;
  if ((st = f32_adapters(a, op_ptrs, ranks, scales, n_adapters))) return st;
  if (op_layout != 0 && op_layout != 1) return MLORA_ERR_INVALID;
  const int rmax = f32_max_rank(a);
  if (width < rmax) return MLORA_ERR_INVALID;
  if ((st = check_f32_matrix(p, ldp, M, K))) return st;
  if ((st = check_f32_matrix(h, ldh, M, width))) return st;
  if (M == 0 || width == 0) return MLORA_OK;
  for (int i = 0; i < kMaxAdapters; ++i) {
    // layout 0: Op_a [r, K] (Q(j, k) = Op[j·K + k]); layout 1: Op_a [K, r] (Q(j, k) = Op[k·r + j])
    a.qe_sr[i] = op_layout == 0 ? K : 1;
    a.qe_sk[i] = op_layout == 0 ? 1 : a.rank[i];
  }
  a.P = static_cast<const float *>(p);
  a.ldp = ldp;
  a.C = static_cast<float *>(h);
  a.ldc = ldh;
  a.M = (int32_t)M;
  a.Kc = (int32_t)K;
  a.Ncols = (int32_t)width;
  a.shrink = 1;
  return f32_launch_linear(a, op_layout == 0, static_cast<hipStream_t>(stream));
}

extern "C" int mlora_f32_gemm_fwd(const void *x, int64_t ldx, int64_t M, int64_t K, const void *w, int64_t ldw,
                                  int64_t N, const void *bias, const void *h_rows, int64_t ldh,
                                  const void *const *b_ptrs, const int32_t *ranks, int32_t n_adapters,
                                  const int64_t *seg_offsets, const int32_t *adapter_ids, int32_t n_segments, void *y,
                                  int64_t ldy, void *stream) {
  F32LinArgs a{};
  if (!f32_dims_ok(M, K, N)) return MLORA_ERR_LIMIT;
  int st = build_segtable(a.seg, M, seg_offsets, adapter_ids, n_segments, n_adapters);
  if (st) return st;
  if ((st = f32_adapters(a, b_ptrs, ranks, nullptr, n_adapters))) return st;
  const int rmax = f32_max_rank(a);
  if ((st = check_f32_matrix(x, ldx, M, K))) return st;
  if ((st = check_f32_matrix(w, ldw, N, K))) return st;
  if ((st = check_f32_matrix(y, ldy, M, N))) return st;
  if (rmax > 0 && (st = check_f32_matrix(h_rows, ldh, M, rmax))) return st;
  if (bias != nullptr && !aligned4(bias)) return MLORA_ERR_UNSUPPORTED;
  if (M == 0 || N == 0) return MLORA_OK;
  for (int i = 0; i < kMaxAdapters; ++i) {  // B_a [N, r]: Q(j = n, k = j') = B[n·r + j']
    a.qe_sr[i] = a.rank[i];
    a.qe_sk[i] = 1;
  }
  a.P = static_cast<const float *>(x);
  a.ldp = ldx;
  a.Q = static_cast<const float *>(w);
  a.q_sr = ldw;
  a.q_sk = 1;
  a.E = static_cast<const float *>(h_rows);
  a.lde = ldh;
  a.bias = static_cast<const float *>(bias);
  a.C = static_cast<float *>(y);
  a.ldc = ldy;
  a.M = (int32_t)M;
  a.Kc = (int32_t)K;
  a.Ncols = (int32_t)N;
  return f32_launch_linear(a, true, static_cast<hipStream_t>(stream));
}

extern "C" int mlora_f32_gemm_dx(const void *dy, int64_t lddy, int64_t M, int64_t N, const void *w, int64_t ldw,
                                 int64_t K, const void *g_rows, int64_t ldg, const void *const *a_ptrs,
                                 const int32_t *ranks, int32_t n_adapters, const int64_t *seg_offsets,
                                 const int32_t *adapter_ids, int32_t n_segments, void *dx, int64_t lddx,
                                 void *stream) {
  F32LinArgs a{};
  if (!f32_dims_ok(M, N, K)) return MLORA_ERR_LIMIT;
  int st = build_segtable(a.seg, M, seg_offsets, adapter_ids, n_segments, n_adapters);
  if (st) return st;
  if ((st = f32_adapters(a, a_ptrs, ranks, nullptr, n_adapters))) return st;
  const int rmax = f32_max_rank(a);
  if ((st = check_f32_matrix(dy, lddy, M, N))) return st;
  if ((st = check_f32_matrix(w, ldw, N, K))) return st;
  if ((st = check_f32_matrix(dx, lddx, M, K))) return st;
  if (rmax > 0 && (st = check_f32_matrix(g_rows, ldg, M, rmax))) return st;
  if (M == 0 || K == 0) return MLORA_OK;
  for (int i = 0; i < kMaxAdapters; ++i) {  // A_a [r, K]: Q(j = k', k = j') = A[j'·K + k']
    a.qe_sr[i] = 1;
    a.qe_sk[i] = K;
  }
  a.P = static_cast<const float *>(dy);
  a.ldp = lddy;
  a.Q = static_cast<const float *>(w);  // W [N, K]: Q(j = k', k = n) = W[n·ldw + k']
  a.q_sr = 1;
  a.q_sk = ldw;
  a.E = static_cast<const float *>(g_rows);
  a.lde = ldg;
  a.bias = nullptr;
  a.C = static_cast<float *>(dx);
  a.ldc = lddx;
  a.M = (int32_t)M;
  a.Kc = (int32_t)N;
  a.Ncols = (int32_t)K;
  return f32_launch_linear(a, false, static_cast<hipStream_t>(stream));
}

extern "C" int mlora_f32_seg_outer(const void *p, int64_t ldp, int64_t M, int64_t C, const void *h, int64_t ldh,
                                   void *const *out_ptrs, int out_layout, const int32_t *ranks, int32_t n_adapters,
                                   const int64_t *seg_offsets, const int32_t *adapter_ids, int32_t n_segments,
                                   void *stream) {
  F32OuterArgs a{};
  if (!f32_dims_ok(M, C, 0)) return MLORA_ERR_LIMIT;
  int st = build_segtable(a.seg, M, seg_offsets, adapter_ids, n_segments, n_adapters);
  if (st) return st;
  if (out_layout != 0 && out_layout != 1) return MLORA_ERR_INVALID;
  if (n_adapters < 0) return MLORA_ERR_INVALID;
  if (n_adapters > kMaxAdapters) return MLORA_ERR_LIMIT;
  if (n_adapters > 0 && (ranks == nullptr || out_ptrs == nullptr)) return MLORA_ERR_INVALID;
  int rmax = 0;
  for (int i = 0; i < kMaxAdapters; ++i) {
    a.rank[i] = 0;
    a.out[i] = nullptr;
  }
  for (int i = 0; i < n_adapters; ++i) {
    if (ranks[i] < 0) return MLORA_ERR_INVALID;
    if (ranks[i] > kMaxRank) return MLORA_ERR_LIMIT;
    a.rank[i] = ranks[i];
    a.out[i] = static_cast<float *>(out_ptrs[i]);
    if (ranks[i] > 0 && C > 0 && (a.out[i] == nullptr || !aligned4(a.out[i]))) return MLORA_ERR_INVALID;
    rmax = ranks[i] > rmax ? ranks[i] : rmax;
  }
  if ((st = check_f32_matrix(p, ldp, M, C))) return st;
  if ((st = check_f32_matrix(h, ldh, M, rmax))) return st;
  if (C == 0 || rmax == 0) return MLORA_OK;
  a.P = static_cast<const float *>(p);
  a.ldp = ldp;
  a.H = static_cast<const float *>(h);
  a.ldh = ldh;
  a.Ci = (int32_t)C;
  a.out_layout = out_layout;
  const int64_t ti = (C + FB - 1) / FB, tj = (rmax + FB - 1) / FB;
  a.tiles_j = (int32_t)tj;
  hipLaunchKernelGGL(f32_outer_kernel, dim3((unsigned)(ti * tj), (unsigned)n_adapters), dim3(256), 0,
                     static_cast<hipStream_t>(stream), a);
  return launch_status();
}
