// Base-projection GEMMs of the multi-LoRA linear, with the LoRA term fused in.
//
//   forward : Y[m,n]  = bf16( Σ_k X[m,k]·W[n,k]  + bias[n] + Σ_j Hs[m,j]·B_a[n,j] )
//   dX      : dX[m,k] = bf16( Σ_n dY[m,n]·W[n,k]            + Σ_j Gs[m,j]·A_a[j,k] )
//
// Both are C = P·Q with P row-major [M, Kc] (contraction contiguous) and Q
// either "NT" ([Ncols, Kc], contraction contiguous: W in the forward, B_a) or
// "NN" ([Kc, Ncols]: W and A_a in dX). The LoRA term is more contraction: after
// the main loop over Kc, every segment that overlaps the tile's rows and has
// an adapter runs ceil(r/64) extra k-tiles with P = Hs rows of that segment
// (other rows read as zero) and Q = that adapter's B_a / A_a. Y is written once.
//
// gfx950 mapping: v_mfma_f32_32x32x16_bf16, wave64. A workgroup of WM x WN
// waves owns a BM x BN tile; each wave a (BM/WM) x (BN/WN) sub-tile whose fp32
// accumulators live in AGPRs. Operand tiles of 64 contraction elements are
// double-buffered in LDS (one barrier per k-tile): the buffer loads of tile k+1
// are in flight while tile k is multiplied. Global reads use raw buffer
// resources; out-of-range rows/columns are given an offset past the buffer and
// read as zero, so tails need no branches. NN operands are transposed in
// registers (8x8 blocks of bf16) on their way into LDS, so both layouts are
// read from LDS the same way (16-byte fragments, XOR-swizzled chunks).
// Reference semantics: training/low_rank.py:26-28 (and its autograd backward).
#include "mlora_common.h"
#include "mlora_host.h"

namespace mlora {

struct GemmArgs {
  const uint16_t *P;
  const uint16_t *Q;
  const uint16_t *E;  // extension rows (Hs / Gs), [M, lde]
  const void *bias;
  uint16_t *Y;
  int64_t ldp, ldq, lde, ldy;
  int32_t M, Ncols, Kc;
  int32_t bias_dtype;  // -1: none
  int32_t accumulate;
  int32_t tiles_m, tiles_n;
  AdapterTable ext;  // NT: B_a [Ncols, r]; NN: A_a [r, Ncols]
  SegTable seg;
};

template <int BM_, int BN_, int WM_, int WN_, bool NN_>
struct GemmCfg {
  static constexpr int BM = BM_, BN = BN_, WM = WM_, WN = WN_;
  static constexpr bool NN = NN_;
  static constexpr int BK = 64;
  static constexpr int THREADS = 64 * WM * WN;
  static constexpr int TM = BM / WM / 32;  // 32x32 MFMA tiles per wave along m
  static constexpr int TN = BN / WN / 32;  // ... along n
  static constexpr int A_CH = BM * 8 / THREADS;  // 16-byte chunks of the P tile per thread
  static constexpr int B_CH = BN * 8 / THREADS;  // NT: chunks of the Q tile per thread
  static constexpr int B_BLK = (BN + THREADS - 1) / THREADS;  // NN: 8x8 blocks per thread
  static constexpr int ROWS_PER_PASS = THREADS / 8;
  static constexpr int STAGE = (BM + BN) * 8;  // u32x4 per LDS stage
  static_assert(A_CH * THREADS == BM * 8, "P tile must split evenly over threads");
  static_assert(NN || B_CH * THREADS == BN * 8, "Q tile must split evenly over threads");
  static constexpr int GROUP_M = 8;
};

// One contraction source (wave-uniform): P rows valid in [row_lo, row_hi),
// contraction valid below klim for both operands.
struct KSource {
  const uint16_t *P;
  const uint16_t *Q;
  int64_t ldp, ldq;
  int32_t row_lo, row_hi;
  int32_t klim;
};

template <class C>
struct Pipe {
  __amdgpu_buffer_rsrc_t rp, rq;
  int32_t p_off[C::A_CH];  // byte offset of each P chunk at k = 0, or kOOB
  int32_t q_off[C::NN ? 1 : C::B_CH];
  int32_t kchunk;          // 8 * (tid & 7): contraction index of this thread's chunks
  int32_t ldq_b;
  int32_t nn_col_ok;
  int32_t klim;
  u32x4 a_regs[C::A_CH];
  u32x4 b_regs[C::NN ? 8 * C::B_BLK : C::B_CH];

  __device__ __forceinline__ void init(const KSource &s, int m0, int n0, int Ncols, int tid) {
    klim = s.klim;
    kchunk = 8 * (tid & 7);
    const int base_row = max(s.row_lo, m0);
    const int64_t ldp_b = s.ldp * 2;
    rp = make_rsrc(s.P + (int64_t)base_row * s.ldp, (int64_t)(s.row_hi - base_row) * ldp_b);
#pragma unroll
    for (int i = 0; i < C::A_CH; ++i) {
      const int grow = m0 + (tid >> 3) + i * C::ROWS_PER_PASS;
      p_off[i] = (grow >= base_row && grow < s.row_hi) ? (int32_t)((grow - base_row) * ldp_b + kchunk * 2) : kOOB;
    }
    ldq_b = (int32_t)(s.ldq * 2);
    if constexpr (!C::NN) {
      rq = make_rsrc(s.Q + (int64_t)n0 * s.ldq, (int64_t)(Ncols - n0) * s.ldq * 2);
#pragma unroll
      for (int i = 0; i < C::B_CH; ++i) q_off[i] = ((tid >> 3) + i * C::ROWS_PER_PASS) * ldq_b + kchunk * 2;
    } else {
      rq = make_rsrc(s.Q + n0, (int64_t)s.klim * s.ldq * 2);
      const int bc = tid % (C::BN / 8);
      nn_col_ok = (n0 + 8 * bc < Ncols) ? 1 : 0;
    }
  }

  __device__ __forceinline__ void load(int k0, int tid) {
    const bool kok = k0 + kchunk < klim;
#pragma unroll
    for (int i = 0; i < C::A_CH; ++i) a_regs[i] = buf_load16(rp, kok ? p_off[i] + k0 * 2 : kOOB);
    if constexpr (!C::NN) {
#pragma unroll
      for (int i = 0; i < C::B_CH; ++i) b_regs[i] = buf_load16(rq, kok ? q_off[i] + k0 * 2 : kOOB);
    } else {
#pragma unroll
      for (int i = 0; i < C::B_BLK; ++i) {
        const int b = tid + i * C::THREADS;
        const int a = b / (C::BN / 8), bc = b % (C::BN / 8);
        const bool ok = b < C::BN && nn_col_ok;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const int kr = k0 + a * 8 + e;
          b_regs[i * 8 + e] = buf_load16(rq, (ok && kr < klim) ? kr * ldq_b + bc * 16 : kOOB);
        }
      }
    }
  }

  __device__ __forceinline__ void store(lds_u4 *ldsA, lds_u4 *ldsB, int tid) const {
    const int c = tid & 7;
#pragma unroll
    for (int i = 0; i < C::A_CH; ++i) {
      const int r = (tid >> 3) + i * C::ROWS_PER_PASS;
      ldsA[lds_chunk_offset(r, c)] = a_regs[i];
    }
    if constexpr (!C::NN) {
#pragma unroll
      for (int i = 0; i < C::B_CH; ++i) {
        const int r = (tid >> 3) + i * C::ROWS_PER_PASS;
        ldsB[lds_chunk_offset(r, c)] = b_regs[i];
      }
    } else {
#pragma unroll
      for (int i = 0; i < C::B_BLK; ++i) {
        const int b = tid + i * C::THREADS;
        if (b < C::BN) {
          const int a = b / (C::BN / 8), bc = b % (C::BN / 8);
          u32x4 blk[8], tr[8];
#pragma unroll
          for (int e = 0; e < 8; ++e) blk[e] = b_regs[i * 8 + e];
          transpose8x8_b16(blk, tr);
#pragma unroll
          for (int t = 0; t < 8; ++t) ldsB[lds_chunk_offset(bc * 8 + t, a)] = tr[t];
        }
      }
    }
  }
};

template <class C>
__device__ __forceinline__ void mma_stage(f32x16 (&acc)[C::TM][C::TN], const lds_u4 *ldsA, const lds_u4 *ldsB,
                                          int wm0, int wn0, int lane) {
#pragma unroll
  for (int s = 0; s < 4; ++s) {
    const int c = 2 * s + (lane >> 5);
    bf16x8 af[C::TM], bf[C::TN];
#pragma unroll
    for (int i = 0; i < C::TM; ++i) af[i] = as_bf16x8(ldsA[lds_chunk_offset(wm0 + 32 * i + (lane & 31), c)]);
#pragma unroll
    for (int j = 0; j < C::TN; ++j) bf[j] = as_bf16x8(ldsB[lds_chunk_offset(wn0 + 32 * j + (lane & 31), c)]);
#pragma unroll
    for (int i = 0; i < C::TM; ++i)
#pragma unroll
      for (int j = 0; j < C::TN; ++j)
        // MFMA rows <- Q (n), columns <- P (m): each lane ends up with 4
        // consecutive n of one row m, stored as one 8-byte write.
        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(bf[j], af[i], acc[i][j], 0, 0, 0);
  }
}

// Contraction over one source, pipelined through the two LDS stages.
template <class C>
__device__ __forceinline__ void run_source(f32x16 (&acc)[C::TM][C::TN], const KSource &src, lds_u4 *lds, int m0,
                                           int n0, int Ncols, int wm0, int wn0, int tid, int lane) {
  const int nk = (src.klim + C::BK - 1) / C::BK;
  if (nk <= 0) return;
  Pipe<C> pipe;
  pipe.init(src, m0, n0, Ncols, tid);
  pipe.load(0, tid);
  __syncthreads();  // LDS may still be read by a previous source's last stage
  pipe.store(lds, lds + C::BM * 8, tid);
  __syncthreads();
  for (int kt = 0; kt < nk; ++kt) {
    // the load past the last tile reads zeros (offsets out of range) and is never used
    pipe.load((kt + 1) * C::BK, tid);
    // keep the loads issued ahead of the MFMAs (the scheduler would sink them
    // next to their LDS stores and expose the full memory latency)
    __builtin_amdgcn_sched_barrier(0);
    lds_u4 *cur = lds + (kt & 1) * C::STAGE;
    lds_u4 *nxt = lds + ((kt + 1) & 1) * C::STAGE;
    mma_stage<C>(acc, cur, cur + C::BM * 8, wm0, wn0, lane);
    __builtin_amdgcn_sched_barrier(0);
    pipe.store(nxt, nxt + C::BM * 8, tid);
    __syncthreads();
  }
}

template <class C>
__global__ __launch_bounds__(C::THREADS) void gemm_kernel(const GemmArgs args) {
  __shared__ u32x4 smem[2 * C::STAGE];
  lds_u4 *lds = (lds_u4 *)smem;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm0 = (wave / C::WN) * (C::BM / C::WM);
  const int wn0 = (wave % C::WN) * (C::BN / C::WN);

  // Tile order: XCD-contiguous ids, then groups of GROUP_M row-tiles walked
  // column by column so concurrently running tiles share P rows and Q columns in L2.
  const int nblocks = args.tiles_m * args.tiles_n;
  const int id = xcd_remap(blockIdx.x, nblocks);
  const int per_group = C::GROUP_M * args.tiles_n;
  const int group = id / per_group;
  const int first_m = group * C::GROUP_M;
  const int gsize = min(args.tiles_m - first_m, C::GROUP_M);
  const int tm = first_m + (id % per_group) % gsize;
  const int tn = (id % per_group) / gsize;
  const int m0 = tm * C::BM, n0 = tn * C::BN;

  f32x16 acc[C::TM][C::TN];
#pragma unroll
  for (int i = 0; i < C::TM; ++i)
#pragma unroll
    for (int j = 0; j < C::TN; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.f;

  // main contraction
  {
    KSource src{args.P, args.Q, args.ldp, args.ldq, 0, args.M, args.Kc};
    run_source<C>(acc, src, lds, m0, n0, args.Ncols, wm0, wn0, tid, lane);
  }
  // LoRA term: one pass per overlapping segment that has an adapter
  if (args.E != nullptr) {
    const int row_end = min(m0 + C::BM, args.M);
    for (int s = seg_of_row(args.seg, m0); s < args.seg.n && args.seg.off[s] < row_end; ++s) {
      const int a = args.seg.aid[s];
      if (a < 0) continue;
      const int r = args.ext.rank[a];
      const int lo = max(args.seg.off[s], m0), hi = min(args.seg.off[s + 1], row_end);
      if (r == 0 || lo >= hi) continue;
      KSource src{args.E, args.ext.ptr[a], args.lde, C::NN ? (int64_t)args.Ncols : (int64_t)r, lo, hi, r};
      run_source<C>(acc, src, lds, m0, n0, args.Ncols, wm0, wn0, tid, lane);
    }
  }

  // epilogue: + bias, (+ Y), round to bf16, 8-byte stores of 4 consecutive n
  const int rows_here = min(C::BM, args.M - m0);
  const int64_t ldy_b = args.ldy * 2;
  const __amdgpu_buffer_rsrc_t ry = make_rsrc(args.Y + (int64_t)m0 * args.ldy, rows_here * ldy_b);
#pragma unroll
  for (int i = 0; i < C::TM; ++i) {
    const int ml = wm0 + 32 * i + (lane & 31);
    if (ml >= rows_here) continue;
#pragma unroll
    for (int j = 0; j < C::TN; ++j) {
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int n = n0 + wn0 + 32 * j + 8 * g + 4 * (lane >> 5);
        if (n >= args.Ncols) continue;
        float v[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] = acc[i][j][4 * g + e];
        if (args.bias_dtype == MLORA_F32) {
          const float4 b = *reinterpret_cast<const float4 *>(static_cast<const float *>(args.bias) + n);
          v[0] += b.x; v[1] += b.y; v[2] += b.z; v[3] += b.w;
        } else if (args.bias_dtype == MLORA_BF16) {
          const uint2 b = *reinterpret_cast<const uint2 *>(static_cast<const uint16_t *>(args.bias) + n);
          v[0] += bf16_to_f32(b.x & 0xffff); v[1] += bf16_to_f32(b.x >> 16);
          v[2] += bf16_to_f32(b.y & 0xffff); v[3] += bf16_to_f32(b.y >> 16);
        }
        const int32_t off = (int32_t)(ml * ldy_b + n * 2);
        if (args.accumulate) {
          const uint2 o = *reinterpret_cast<const uint2 *>(args.Y + (int64_t)(m0 + ml) * args.ldy + n);
          v[0] += bf16_to_f32(o.x & 0xffff); v[1] += bf16_to_f32(o.x >> 16);
          v[2] += bf16_to_f32(o.y & 0xffff); v[3] += bf16_to_f32(o.y >> 16);
        }
        buf_store8(ry, off, make_uint2(pack2_bf16(v[0], v[1]), pack2_bf16(v[2], v[3])));
      }
    }
  }
}

using CfgNT256 = GemmCfg<256, 256, 2, 2, false>;
using CfgNN256 = GemmCfg<256, 256, 2, 2, true>;
using CfgNT128 = GemmCfg<128, 128, 2, 2, false>;
using CfgNN128 = GemmCfg<128, 128, 2, 2, true>;

template <class C>
static int launch_gemm(GemmArgs &a, hipStream_t stream) {
  a.tiles_m = (a.M + C::BM - 1) / C::BM;
  a.tiles_n = (a.Ncols + C::BN - 1) / C::BN;
  const int64_t nblocks = (int64_t)a.tiles_m * a.tiles_n;
  if (nblocks == 0) return MLORA_OK;
  if (nblocks > INT32_MAX) return MLORA_ERR_LIMIT;
  hipLaunchKernelGGL(gemm_kernel<C>, dim3((unsigned)nblocks), dim3(C::THREADS), 0, stream, a);
  return launch_status();
}

// Tile choice: 256x256 when that still gives every CU at least one tile, else 128x128.
template <class Big, class Small>
static int dispatch_gemm(GemmArgs &a, hipStream_t stream) {
  const int64_t big_tiles = (int64_t)((a.M + 255) / 256) * ((a.Ncols + 255) / 256);
  if (big_tiles >= 256) return launch_gemm<Big>(a, stream);
  return launch_gemm<Small>(a, stream);
}

static int fill_common(GemmArgs &a, int64_t M, int64_t Kc, int64_t Ncols, const void *e, int64_t lde,
                       const void *const *ext_ptrs, const int32_t *ranks, int32_t n_adapters, const int64_t *seg_offsets,
                       const int32_t *adapter_ids, int32_t n_segments) {
  if (M < 0 || Kc < 0 || Ncols < 0) return MLORA_ERR_INVALID;
  if (M > INT32_MAX - 1024 || Kc > INT32_MAX - 1024 || Ncols > INT32_MAX - 1024) return MLORA_ERR_LIMIT;
  int st = build_segtable(a.seg, M, seg_offsets, adapter_ids, n_segments, n_adapters);
  if (st) return st;
  st = build_adapters(a.ext, a.seg, ext_ptrs, ranks, nullptr, n_adapters);
  if (st) return st;
  const int rmax = max_used_rank(a.seg, a.ext);
  if (rmax > 0) {
    st = check_bf16_matrix(e, lde, M, rmax);
    if (st) return st;
  }
  a.E = rmax > 0 ? static_cast<const uint16_t *>(e) : nullptr;
  a.lde = lde;
  a.M = (int32_t)M;
  a.Kc = (int32_t)Kc;
  a.Ncols = (int32_t)Ncols;
  return MLORA_OK;
}

// Byte offsets inside one buffer resource are 31-bit: a tile's rows of P and Y,
// and all of an NN operand, must stay below that.
static bool offsets_fit(int64_t ld, int64_t rows) { return ld * 2 * rows < (int64_t)kOOB; }

}  // namespace mlora

using namespace mlora;

extern "C" int mlora_gemm_fwd(const void *x, int64_t ldx, int64_t M, int64_t K, const void *w, int64_t ldw, int64_t N,
                              const void *bias, int bias_dtype, const void *h_rows, int64_t ldh,
                              const void *const *b_ptrs, const int32_t *ranks, int32_t n_adapters,
                              const int64_t *seg_offsets, const int32_t *adapter_ids, int32_t n_segments, void *y,
                              int64_t ldy, int accumulate, void *stream) {
  GemmArgs a{};
  int st = fill_common(a, M, K, N, h_rows, ldh, b_ptrs, ranks, n_adapters, seg_offsets, adapter_ids, n_segments);
  if (st) return st;
  if ((st = check_bf16_matrix(x, ldx, M, K))) return st;
  if ((st = check_bf16_matrix(w, ldw, N, K))) return st;
  if ((st = check_bf16_matrix(y, ldy, M, N))) return st;
  if (M == 0 || N == 0) return MLORA_OK;
  if (y == nullptr) return MLORA_ERR_INVALID;
  if (bias != nullptr) {
    if (bias_dtype != MLORA_F32 && bias_dtype != MLORA_BF16) return MLORA_ERR_UNSUPPORTED;
    if (!aligned16(bias)) return MLORA_ERR_UNSUPPORTED;
  }
  if (!offsets_fit(ldx, 256) || !offsets_fit(ldy, 256) || !offsets_fit(ldw, 256)) return MLORA_ERR_LIMIT;
  a.P = static_cast<const uint16_t *>(x);
  a.Q = static_cast<const uint16_t *>(w);
  a.ldp = ldx;
  a.ldq = ldw;
  a.bias = bias;
  a.bias_dtype = bias ? bias_dtype : -1;
  a.Y = static_cast<uint16_t *>(y);
  a.ldy = ldy;
  a.accumulate = accumulate ? 1 : 0;
  return dispatch_gemm<CfgNT256, CfgNT128>(a, static_cast<hipStream_t>(stream));
}

extern "C" int mlora_gemm_dx(const void *dy, int64_t lddy, int64_t M, int64_t N, const void *w, int64_t ldw, int64_t K,
                             const void *g_rows, int64_t ldg, const void *const *a_ptrs, const int32_t *ranks,
                             int32_t n_adapters, const int64_t *seg_offsets, const int32_t *adapter_ids,
                             int32_t n_segments, void *dx, int64_t lddx, void *stream) {
  GemmArgs a{};
  // contraction over N, output columns K
  int st = fill_common(a, M, N, K, g_rows, ldg, a_ptrs, ranks, n_adapters, seg_offsets, adapter_ids, n_segments);
  if (st) return st;
  if ((st = check_bf16_matrix(dy, lddy, M, N))) return st;
  if ((st = check_bf16_matrix(w, ldw, N, K))) return st;
  if ((st = check_bf16_matrix(dx, lddx, M, K))) return st;
  if (M == 0 || K == 0) return MLORA_OK;
  if (dx == nullptr) return MLORA_ERR_INVALID;
  if (!offsets_fit(lddy, 256) || !offsets_fit(lddx, 256) || !offsets_fit(ldw, N) || !offsets_fit(K, kMaxRank))
    return MLORA_ERR_LIMIT;
  a.P = static_cast<const uint16_t *>(dy);
  a.Q = static_cast<const uint16_t *>(w);
  a.ldp = lddy;
  a.ldq = ldw;
  a.bias = nullptr;
  a.bias_dtype = -1;
  a.Y = static_cast<uint16_t *>(dx);
  a.ldy = lddx;
  a.accumulate = 0;
  return dispatch_gemm<CfgNN256, CfgNN128>(a, static_cast<hipStream_t>(stream));
}
