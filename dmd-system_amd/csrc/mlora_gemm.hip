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
// accumulators stay in registers. Operand tiles of 64 contraction elements are
// double-buffered in LDS (one barrier per k-tile): the direct-to-LDS loads of
// tile k+1 are issued one by one between the MFMAs of tile k. Global reads use raw buffer
// resources; out-of-range rows/columns are given an offset past the buffer and
// read as zero, so tails need no branches. NN operands stay in their natural
// layout in LDS and are read with the gfx950 transposing LDS read
// (ds_read_b64_tr_b16), which turns 4 rows x 4 columns into per-column
// contraction runs, i.e. MFMA B fragments.
// Reference semantics: training/low_rank.py:26-28 (and its autograd backward).
#include "mlora_common.h"
#include "mlora_host.h"

#include <type_traits>

namespace mlora {

struct GemmArgs {
  const void *P;       // bf16, or e4m3 in the fp8 forward
  const void *Q;       // bf16, or e4m3 in the fp8 forward
  const uint16_t *E;   // extension rows (Hs / Gs), [M, lde]
  const float *psc;    // fp8 forward: per-row scale of P [M]
  const float *qsc;    // fp8 forward: per-row scale of Q [Ncols]
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

template <int BM_, int BN_, int WM_, int WN_, bool NN_, bool F8_ = false>
struct GemmCfg {
  static constexpr int BM = BM_, BN = BN_, WM = WM_, WN = WN_;
  static constexpr bool NN = NN_;
  static constexpr bool F8 = F8_;  // main contraction in e4m3 (v_mfma_scale_f32_32x32x64_f8f6f4)
  static_assert(!(NN && F8), "the fp8 main contraction is NT only");
  static constexpr int NW = WM * WN;
  static constexpr int THREADS = 64 * NW;
  static constexpr int TM = BM / WM / 32;  // 32x32 MFMA tiles per wave along m
  static constexpr int TN = BN / WN / 32;  // ... along n
  static constexpr int A_DMA = BM / 8 / NW;  // 1 KB direct-to-LDS loads per wave for the P tile
  static constexpr int B_DMA = BN / 8 / NW;  // the same for the Q tile (both layouts hold 64 x BN)
  // NN Q tile: natural layout, one row of BN output columns per contraction index
  static constexpr int QROW = BN * 2;       // bytes per NN row
  static constexpr int QCPR = BN / 8;       // 16-byte chunks per NN row
  static constexpr int QRPD = 1024 / QROW;  // NN rows per 1 KB load
  static_assert(A_DMA * NW * 8 == BM, "P tile rows must split into 8-row loads over the waves");
  static_assert(B_DMA * NW * 8 == BN, "Q tile must split into 1 KB loads over the waves");
  static_assert(A_DMA % 2 == 0 && B_DMA % 2 == 0, "even 1 KB load counts per wave");
  static_assert(!NN || (QCPR >= 16 && QRPD >= 1), "NN rows hold at least 16 chunks");
  static constexpr int NDMA = A_DMA + B_DMA;  // 1 KB loads per wave and k-tile
  static constexpr int TMN = TM * TN;         // MFMAs per wave and 16-deep substep
  // The next tile's loads are spread over the MFMAs of this tile's first two
  // substeps, one after every DMA_EVERY-th MFMA (the stage barrier after the
  // last substep waits for them).
  static constexpr int DMA_EVERY = 2 * TMN / NDMA > 1 ? 2 * TMN / NDMA : 1;
  static_assert(NDMA * DMA_EVERY <= (F8 ? 2 : 4) * TMN, "every load is issued within the k-tile");
  // LDS (bytes): P stage 0 | P stage 1 | Q stage 0 | Q stage 1
  static constexpr int A_BYTES = BM * 128, B_BYTES = BN * 128;
  static constexpr int B_BASE = 2 * A_BYTES;
  static constexpr int LDS_BYTES = 2 * (A_BYTES + B_BYTES);
  static_assert(A_BYTES < 65536 && B_BYTES < 65536, "stage offsets must fit the ds_read offset field");
  static constexpr int GROUP_M = 8;
};

// One contraction source (wave-uniform): P rows valid in [row_lo, row_hi),
// contraction valid below klim (elements) for both operands. esz is the
// element size (2: bf16, 1: e4m3); an LDS k-tile always holds 128 bytes of
// contraction per row, i.e. 128 / esz elements.
struct KSource {
  const char *P;
  const char *Q;
  int64_t ldp_b, ldq_b;  // row pitches in bytes
  int32_t row_lo, row_hi;
  int32_t klim;
  int32_t esz;
};

// Per-thread state of one contraction source. Global tiles go to LDS with the
// gfx950 direct-to-LDS buffer load: one wave instruction fills 1 KB (8 rows of
// 8 chunks); lane L lands at chunk slot L of that KB, so it fetches the
// logical chunk (L%8) ^ swz(row) that the XOR-swizzled layout keeps there.
// With swz depending on row%16 only, the 1 KB loads of one wave differ by a
// whole number of rows plus one of two lane patterns (even / odd 8-row block),
// so the per-load row step and the tile's k offset travel in soffset.
template <class C>
struct Pipe {
  __amdgpu_buffer_rsrc_t rp, rq;
  int32_t a_off[2];     // even / odd 8-row block: this lane's P chunk offset at k = 0 (rows past the tile: kOOB)
  int32_t a_kc[2];      // contraction index of that chunk
  int32_t a_row0;       // first P row (tile-local) of this wave's loads
  int32_t b_off[2], b_kc[2];
  int32_t b_row0;
  int32_t klim, ldp_b, ldq_b, p_rows, esz;

  __device__ __forceinline__ void init(const KSource &s, int m0, int n0, int Ncols, int tid) {
    const int lane = tid & 63, wave = wave_id();
    klim = s.klim;
    esz = s.esz;
    const int base_row = max(s.row_lo, m0);
    ldp_b = (int32_t)s.ldp_b;
    ldq_b = (int32_t)s.ldq_b;
    const int chunk_elems = 16 / s.esz;
    // P rows of the tile are read relative to m0; rows outside [row_lo, row_hi) read zero
    rp = make_rsrc(s.P + (int64_t)m0 * s.ldp_b, (int64_t)(s.row_hi - m0) * ldp_b);
    p_rows = base_row - m0;  // tile rows below this index belong to another segment
    a_row0 = 8 * wave * C::A_DMA;
#pragma unroll
    for (int par = 0; par < 2; ++par) {
      const int c = (lane & 7) ^ (lane >> 3) ^ par;
      a_kc[par] = chunk_elems * c;
      a_off[par] = (lane >> 3) * ldp_b + 16 * c;
    }
    if constexpr (!C::NN) {
      rq = make_rsrc(s.Q + (int64_t)n0 * s.ldq_b, (int64_t)(Ncols - n0) * s.ldq_b);
      b_row0 = 8 * wave * C::B_DMA;
#pragma unroll
      for (int par = 0; par < 2; ++par) {
        const int c = (lane & 7) ^ (lane >> 3) ^ par;
        b_kc[par] = chunk_elems * c;
        b_off[par] = (lane >> 3) * ldq_b + 16 * c;  // rows past Ncols fall outside rq
      }
    } else {
      // NN (bf16 only): rows are contraction indices, chunk c of row k at slot c ^ (4 * (k & 3))
      rq = make_rsrc(s.Q + 2 * n0, (int64_t)s.klim * s.ldq_b);
      const int p = lane % C::QCPR, rl = lane / C::QCPR;
#pragma unroll
      for (int par = 0; par < 2; ++par) {
        const int c = p ^ (4 * ((C::QRPD * par + rl) & 3));
        b_off[par] = (n0 + 8 * c < Ncols) ? rl * ldq_b + 16 * c : kOOB;
      }
      b_kc[0] = rl;  // row of this lane within its 1 KB load
    }
  }

  // Issue 1 KB load number q (of NDMA per wave) of the k-tile starting at k0
  // into LDS stage `st`: q < A_DMA are P rows, the rest Q. live == false turns
  // every lane's offset out of range: the instruction then moves no data.
  __device__ __forceinline__ void issue_one(MLORA_LDS char *lds, int q, int st, int k0, int wave, int lane, bool KMASK,
                                            bool live) const {
    if (q < C::A_DMA) {
      MLORA_LDS void *dst = lds + st * C::A_BYTES + (wave * C::A_DMA + q) * 1024;
      const int row = a_row0 + 8 * q;  // wave-uniform
      const int par = q & 1;
      int32_t off = a_off[par];
      if (p_rows > 0 && row + (lane >> 3) < p_rows) off = kOOB;  // rows of an earlier segment
      if (KMASK && k0 + a_kc[par] >= klim) off = kOOB;
      if (!live) off = kOOB;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rp, dst, 16, off, row * ldp_b + k0 * esz, 0, 0);
    } else if constexpr (!C::NN) {
      const int qb = q - C::A_DMA;
      MLORA_LDS void *dst = lds + C::B_BASE + st * C::B_BYTES + (wave * C::B_DMA + qb) * 1024;
      const int row = b_row0 + 8 * qb;
      const int par = qb & 1;
      int32_t off = (KMASK && k0 + b_kc[par] >= klim) ? kOOB : b_off[par];
      if (!live) off = kOOB;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rq, dst, 16, off, row * ldq_b + k0 * esz, 0, 0);
    } else {
      const int blk = wave * C::B_DMA + (q - C::A_DMA);  // wave-uniform
      MLORA_LDS void *dst = lds + C::B_BASE + st * C::B_BYTES + blk * 1024;
      const int row = C::QRPD * blk;
      int32_t off = (KMASK && k0 + row + b_kc[0] >= klim) ? kOOB : b_off[blk & 1];
      if (!live) off = kOOB;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rq, dst, 16, off, (k0 + row) * ldq_b, 0, 0);
    }
  }

  // All loads of the k-tile starting at k0, back to back (pipeline prologue).
  __device__ __forceinline__ void issue(MLORA_LDS char *lds, int st, int k0, int wave, int lane, bool KMASK) const {
#pragma unroll
    for (int q = 0; q < C::NDMA; ++q) issue_one(lds, q, st, k0, wave, lane, KMASK, true);
  }
};

// Byte addresses (stage 0, first 32-row tile) of this lane's fragments per
// substep; further tiles are +4096 bytes and stage 1 is +A_BYTES / +B_BYTES,
// all folded into the ds_read offset field.
// NN: b[j] is the first of the two transposing reads of tile j at substep 0
// (substep s adds 16 rows, the second read 4 rows). ds_read_b64_tr_b16 gives
// lane j of a 16-lane group element e = element (j & 3) of the 8 bytes
// addressed by lane 4e + (j >> 2); lane i pointing at row k0 + (i >> 2),
// column c0 + 4(i & 3) therefore yields 4 consecutive contraction values of
// column c0 + j: half of the B fragment of v_mfma_f32_32x32x16_bf16.
template <class C>
struct FragAddr {
  int32_t a[4], b[C::NN ? C::TN : 4];
  __device__ __forceinline__ void init(int wm0, int wn0, int lane) {
    const int z = swz(lane & 31);  // lane-constant: fragment rows are 32-aligned + lane
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      const int slot = (2 * s + (lane >> 5)) ^ z;
      a[s] = (wm0 + (lane & 31)) * 128 + 16 * slot;
      if constexpr (!C::NN) b[s] = C::B_BASE + (wn0 + (lane & 31)) * 128 + 16 * slot;
    }
    if constexpr (C::NN) {
      const int i = lane & 15, h = lane >> 5, g1 = (lane >> 4) & 1;
      const int m = (i >> 2) & 3;  // k & 3 of every row this lane reads
#pragma unroll
      for (int j = 0; j < C::TN; ++j) {
        const int c = (wn0 + 32 * j + 16 * g1) / 8 + ((i & 3) >> 1);
        b[j] = C::B_BASE + (8 * h + (i >> 2)) * C::QROW + 16 * (c ^ (4 * m)) + 8 * (i & 1);
      }
    }
  }
};

// Fragment read r of substep s from LDS stage ST: r < TM reads P tile r
// (af[r]), the others Q tile r - TM (bf[r - TM]).
template <class C, int ST>
__device__ __forceinline__ void read_frag(int r, bf16x8 (&af)[C::TM], bf16x8 (&bf)[C::TN], const MLORA_LDS char *lds,
                                          const FragAddr<C> &fa, int s) {
  if (r < C::TM) {
    af[r] = as_bf16x8(*(const lds_u4 *)(lds + fa.a[s] + (4096 * r + ST * C::A_BYTES)));
    return;
  }
  if constexpr (!C::NN) {  // NN Q fragments are read per substep by read_q_nn
    const int j = r - C::TM;
    bf[j] = as_bf16x8(*(const lds_u4 *)(lds + fa.b[s] + (4096 * j + ST * C::B_BYTES)));
  }
}

// All TN Q fragments of substep s of an NN stage: pairs of transposing reads
// (rows 16s + 8h + (i>>2) and 4 rows further) in one block that also waits
// for them (see lds_read_tr16_x4).
template <class C, int ST>
__device__ __forceinline__ void read_q_nn(bf16x8 (&bf)[C::TN], const MLORA_LDS char *lds, const FragAddr<C> &fa,
                                          int s) {
  u32x4 q[C::TN];
  const MLORA_LDS char *base = lds + (ST * C::B_BYTES + 16 * C::QROW * s);
  if constexpr (C::TN == 4) lds_read_tr16_x4<4 * C::QROW>(base, fa.b, q);
  else lds_read_tr16_x2<4 * C::QROW>(base, fa.b, q);
#pragma unroll
  for (int j = 0; j < C::TN; ++j) bf[j] = as_bf16x8(q[j]);
}

// One 64-deep k-tile from LDS stage ST: 4 substeps of 16, entered with the
// substep-0 fragments in af0/bf0 (and leaving the next stage's there). The
// fragments of substep s+1 are read while the TM*TN MFMAs of substep s run,
// and the loads of the next k-tile (into the other stage) are issued between
// the MFMAs, one after every DMA_EVERY-th MFMA: issued back to back they fill
// the texture unit's queue and stall the waves' MFMA issue behind them.
template <class C, int ST>
__device__ __forceinline__ void mma_stage(f32x16 (&acc)[C::TM][C::TN], MLORA_LDS char *lds, const FragAddr<C> &fa,
                                          const Pipe<C> &pipe, int k0, bool kmask, bool live, int wave, int lane) {
  // NN: the TN Q fragments come from read_q_nn (transposing reads + wait, in assembly)
  constexpr int NR = C::NN ? C::TM : C::TM + C::TN;  // compiler-visible fragment reads per substep
  constexpr int DSR = NR;                            // DS read instructions per substep
  bf16x8 af[2][C::TM], bf[2][C::TN];
#pragma unroll
  for (int r = 0; r < NR; ++r) read_frag<C, ST>(r, af[0], bf[0], lds, fa, 0);
  if constexpr (C::NN) read_q_nn<C, ST>(bf[0], lds, fa, 0);
#pragma unroll
  for (int s = 0; s < 4; ++s) {
    const int cur = s & 1;
    if (s < 3) {
#pragma unroll
      for (int r = 0; r < NR; ++r) read_frag<C, ST>(r, af[cur ^ 1], bf[cur ^ 1], lds, fa, s + 1);
      if constexpr (C::NN) read_q_nn<C, ST>(bf[cur ^ 1], lds, fa, s + 1);
    }
#pragma unroll
    for (int g = 0; g < C::TMN; ++g) {
      const int i = g / C::TN, j = g % C::TN;
      // MFMA rows <- Q (n), columns <- P (m): each lane ends up with 4
      // consecutive n of one row m, stored as one 8-byte write.
      acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(bf[cur][j], af[cur][i], acc[i][j], 0, 0, 0);
      const int idx = s * C::TMN + g;
      if (idx % C::DMA_EVERY == 0 && idx / C::DMA_EVERY < C::NDMA)
        pipe.issue_one(lds, idx / C::DMA_EVERY, ST ^ 1, k0, wave, lane, kmask, live);
    }
    // scheduling hints: DS reads spread evenly over the MFMAs, each load right after its MFMA
#pragma unroll
    for (int g = 0; g < C::TMN; ++g) {
      const int nr = s < 3 ? ((g + 1) * DSR) / C::TMN - (g * DSR) / C::TMN : 0;
#pragma unroll
      for (int r = 0; r < nr; ++r) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // one DS read
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);                                // one MFMA
      const int idx = s * C::TMN + g;
      if (idx % C::DMA_EVERY == 0 && idx / C::DMA_EVERY < C::NDMA)
        __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);  // one load
    }
  }
}

// The fp8 form of mma_stage: one 128-element (128-byte) k-tile of e4m3 in 2
// substeps of v_mfma_scale_f32_32x32x64_f8f6f4 (unit block scales). That MFMA
// gives lane l the 32 contraction bytes of row (A) / column (B) l%32 at
// positions 32*(l/32) + e; any assignment of k to (l/32, e) works as long as A
// and B agree, so each operand fragment is simply the two 16-byte chunks that
// the bf16 substeps 2s and 2s+1 read: the LDS layout and addresses are shared.
template <class C, int ST>
__device__ __forceinline__ void mma_stage_fp8(f32x16 (&acc)[C::TM][C::TN], MLORA_LDS char *lds, const FragAddr<C> &fa,
                                              const Pipe<C> &pipe, int k0, bool kmask, bool live, int wave, int lane) {
  typedef int i32x8 __attribute__((ext_vector_type(8)));
  // one 32-byte fragment: P tile r (r < TM) or Q tile r - TM, fp8 substep s
  auto frag = [&](int r, int s) -> i32x8 {
    bf16x8 a[C::TM], b[C::TN];
    read_frag<C, ST>(r, a, b, lds, fa, 2 * s);
    const u32x4 lo = __builtin_bit_cast(u32x4, r < C::TM ? a[r] : b[r - C::TM]);
    read_frag<C, ST>(r, a, b, lds, fa, 2 * s + 1);
    const u32x4 hi = __builtin_bit_cast(u32x4, r < C::TM ? a[r] : b[r - C::TM]);
    return i32x8{(int)lo[0], (int)lo[1], (int)lo[2], (int)lo[3], (int)hi[0], (int)hi[1], (int)hi[2], (int)hi[3]};
  };
  i32x8 ac[C::TM], bc[C::TN], an[C::TM];
#pragma unroll
  for (int i = 0; i < C::TM; ++i) ac[i] = frag(i, 0);
#pragma unroll
  for (int j = 0; j < C::TN; ++j) bc[j] = frag(C::TM + j, 0);
#pragma unroll
  for (int s = 0; s < 2; ++s) {
    if (s == 0) {
#pragma unroll
      for (int i = 0; i < C::TM; ++i) an[i] = frag(i, 1);
    }
    // j-major order: once tile j's MFMAs are issued its fragment is dead and
    // the next substep's fragment of tile j can take its registers
#pragma unroll
    for (int j = 0; j < C::TN; ++j) {
#pragma unroll
      for (int i = 0; i < C::TM; ++i) {
        // MFMA rows <- Q (n), columns <- P (m), as in the bf16 form
        acc[i][j] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(bc[j], ac[i], acc[i][j], 0, 0, 0, 127, 0, 127);
        const int idx = s * C::TMN + j * C::TM + i;
        if (idx % C::DMA_EVERY == 0 && idx / C::DMA_EVERY < C::NDMA)
          pipe.issue_one(lds, idx / C::DMA_EVERY, ST ^ 1, k0, wave, lane, kmask, live);
      }
      if (s == 0) bc[j] = frag(C::TM + j, 1);
    }
    if (s == 0) {
#pragma unroll
      for (int i = 0; i < C::TM; ++i) ac[i] = an[i];
    }
  }
}

// Wait for this wave's direct-to-LDS loads, then publish the stage to all waves.
__device__ __forceinline__ void stage_barrier() {
  __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
  __syncthreads();
}

// Finds the next LoRA source of this tile: the next segment from `seg` on that
// overlaps rows [m0, row_end) and has an adapter. Wave-uniform scalar code.
__device__ __forceinline__ bool next_lora_source(const GemmArgs &args, bool nn, int m0, int row_end, int &seg,
                                                 KSource &src) {
  while (seg < args.seg.n && args.seg.off[seg] < row_end) {
    const int a = args.seg.aid[seg];
    const int lo = max(args.seg.off[seg], m0), hi = min(args.seg.off[seg + 1], row_end);
    ++seg;
    if (a >= 0 && args.ext.rank[a] > 0 && lo < hi) {
      const int r = args.ext.rank[a];
      src = KSource{reinterpret_cast<const char *>(args.E), reinterpret_cast<const char *>(args.ext.ptr[a]), 2 * args.lde,
                    2 * (nn ? (int64_t)args.Ncols : (int64_t)r), lo, hi, r, 2};
      return true;
    }
  }
  return false;
}

// All contraction of one tile in a single pipelined loop over "virtual"
// k-tiles: first the main X·Wᵀ (or dY·W) tiles, then ceil(r/64) tiles per LoRA
// segment overlapping the tile. At a source boundary the loader is re-pointed
// (a few scalars and two offsets); the LDS stages and the MFMA code are shared,
// so the accumulators stay in place. Tiles past a source's contraction length
// mask their chunks.
template <class C>
__device__ __forceinline__ void contract_tile(f32x16 (&acc)[C::TM][C::TN], const GemmArgs &args, MLORA_LDS char *lds,
                                              const FragAddr<C> &fa, int m0, int n0, int tid) {
  const int wave = wave_id(), lane = tid & 63;
  const int row_end = min(m0 + C::BM, args.M);
  int seg = args.E != nullptr ? seg_of_row(args.seg, m0) : args.seg.n;
  Pipe<C> pipe;
  constexpr int esz0 = C::F8 ? 1 : 2;
  KSource src{static_cast<const char *>(args.P), static_cast<const char *>(args.Q), esz0 * args.ldp, esz0 * args.ldq,
              0, args.M, args.Kc, esz0};
  int bk = 128 / src.esz;  // contraction elements per k-tile of the current source
  int ntile = (src.klim + bk - 1) / bk;
  if (ntile == 0) {
    if (!next_lora_source(args, C::NN, m0, row_end, seg, src)) return;
    bk = 128 / src.esz;
    ntile = (src.klim + bk - 1) / bk;
  }
  bool kmask = src.klim % bk != 0;
  pipe.init(src, m0, n0, args.Ncols, tid);
  int t_in_src = 0;  // index of the tile being loaded within its source
  pipe.issue(lds, 0, 0, wave, lane, kmask);
  stage_barrier();
  // `more`: whether a tile after the current one exists (and was loaded)
  auto advance = [&]() -> bool {
    if (++t_in_src < ntile) return true;
    if (!next_lora_source(args, C::NN, m0, row_end, seg, src)) return false;
    bk = 128 / src.esz;
    ntile = (src.klim + bk - 1) / bk;
    kmask = src.klim % bk != 0;
    pipe.init(src, m0, n0, args.Ncols, tid);
    t_in_src = 0;
    return true;
  };
  // One step: multiply the tile in LDS stage ST while the next tile (if any)
  // loads into the other stage; returns whether there is a next tile.
  auto step = [&](auto st_c, auto f8_c) -> bool {
    constexpr int ST = decltype(st_c)::value;
    const bool more = advance();
    if constexpr (decltype(f8_c)::value) mma_stage_fp8<C, ST>(acc, lds, fa, pipe, t_in_src * bk, kmask, more, wave, lane);
    else mma_stage<C, ST>(acc, lds, fa, pipe, t_in_src * bk, kmask, more, wave, lane);
    stage_barrier();
    return more;
  };
  using S0 = std::integral_constant<int, 0>;
  using S1 = std::integral_constant<int, 1>;
  using E4 = std::true_type;
  using B16 = std::false_type;
  if constexpr (C::F8) {
    // the e4m3 main contraction (at least one tile), then the bf16 LoRA tiles
    // (operands pre-divided by the scales) from whichever stage holds the next one
    bool more;
    int st;
    while (true) {
      more = step(S0{}, E4{});
      st = 1;
      if (!more || src.esz != 1) break;
      more = step(S1{}, E4{});
      st = 0;
      if (!more || src.esz != 1) break;
    }
    if (!more) return;
    if (st == 1 && !step(S1{}, B16{})) return;
  }
  while (true) {
    if (!step(S0{}, B16{})) break;
    if (!step(S1{}, B16{})) break;
  }
}

template <class C>
__global__ __launch_bounds__(C::THREADS) void gemm_kernel(const GemmArgs args) {
  __shared__ u32x4 smem[C::LDS_BYTES / 16];
  MLORA_LDS char *lds = (MLORA_LDS char *)smem;
  const int tid = threadIdx.x, lane = tid & 63, wave = wave_id();
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

  // Register 4g + e of tile (i, j) holds row m = m0 + wm0 + 32i + lane%32 and
  // column n = n0 + wn0 + 32j + 8g + 4(lane/32) + e.
  auto bias_of = [&](int n, float (&v)[4]) {
    v[0] = v[1] = v[2] = v[3] = 0.f;
    if (n < args.Ncols) {
      if (args.bias_dtype == MLORA_F32) {
        const f32x4 b = *(const MLORA_GLOBAL f32x4 *)(static_cast<const float *>(args.bias) + n);
        v[0] = b[0]; v[1] = b[1]; v[2] = b[2]; v[3] = b[3];
      } else if (args.bias_dtype == MLORA_BF16) {
        const u32x2 b = *(const MLORA_GLOBAL u32x2 *)(static_cast<const uint16_t *>(args.bias) + n);
        v[0] = bf16_to_f32(b.x & 0xffff); v[1] = bf16_to_f32(b.x >> 16);
        v[2] = bf16_to_f32(b.y & 0xffff); v[3] = bf16_to_f32(b.y >> 16);
      }
    }
  };
  f32x16 acc[C::TM][C::TN];
  if constexpr (!C::F8) {
    // bf16: accumulators start at the bias of their column
#pragma unroll
    for (int j = 0; j < C::TN; ++j) {
      f32x16 b0;
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        float v[4];
        bias_of(n0 + wn0 + 32 * j + 8 * g + 4 * (lane >> 5), v);
#pragma unroll
        for (int e = 0; e < 4; ++e) b0[4 * g + e] = v[e];
      }
#pragma unroll
      for (int i = 0; i < C::TM; ++i) acc[i][j] = b0;
    }
  } else {
#pragma unroll
    for (int i = 0; i < C::TM; ++i)
#pragma unroll
      for (int j = 0; j < C::TN; ++j)
#pragma unroll
        for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.f;
  }
  FragAddr<C> fa;
  fa.init(wm0, wn0, lane);

  contract_tile<C>(acc, args, lds, fa, m0, n0, tid);

  // epilogue: (fp8: scale and bias), (+ Y), round to bf16, 8-byte stores of 4 consecutive n
  const int rows_here = min(C::BM, args.M - m0);
  const int64_t ldy_b = args.ldy * 2;
  const __amdgpu_buffer_rsrc_t ry = make_rsrc(args.Y + (int64_t)m0 * args.ldy, rows_here * ldy_b);
#pragma unroll
  for (int i = 0; i < C::TM; ++i) {
    const int ml = wm0 + 32 * i + (lane & 31);
    float ps = 1.f;
    if constexpr (C::F8) ps = m0 + ml < args.M ? args.psc[m0 + ml] : 0.f;
#pragma unroll
    for (int j = 0; j < C::TN; ++j) {
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int n = n0 + wn0 + 32 * j + 8 * g + 4 * (lane >> 5);
        float v[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] = acc[i][j][4 * g + e];
        if constexpr (C::F8) {
          // acc = Σ xq·wq + Σ (h/x_scale)·(B/w_scale): one scaling restores both, then the bias
          float b[4], qs[4] = {0.f, 0.f, 0.f, 0.f};
          bias_of(n, b);
          if (n < args.Ncols) {
            const f32x4 q = *(const MLORA_GLOBAL f32x4 *)(args.qsc + n);
            qs[0] = q[0]; qs[1] = q[1]; qs[2] = q[2]; qs[3] = q[3];
          }
#pragma unroll
          for (int e = 0; e < 4; ++e) v[e] = v[e] * (ps * qs[e]) + b[e];
        }
        // rows past M / columns past Ncols fall outside ry or are dropped
        const int32_t off = (ml < rows_here && n < args.Ncols) ? (int32_t)(ml * ldy_b + n * 2) : kOOB;
        if (args.accumulate && off != kOOB) {
          const u32x2 o = *(const MLORA_GLOBAL u32x2 *)(args.Y + (int64_t)(m0 + ml) * args.ldy + n);
          v[0] += bf16_to_f32(o.x & 0xffff); v[1] += bf16_to_f32(o.x >> 16);
          v[2] += bf16_to_f32(o.y & 0xffff); v[3] += bf16_to_f32(o.y >> 16);
        }
        buf_store8(ry, off, make_uint2(pack2_bf16(v[0], v[1]), pack2_bf16(v[2], v[3])));
      }
    }
  }
}

using CfgNT256 = GemmCfg<256, 256, 4, 2, false>;
using CfgF8256 = GemmCfg<256, 256, 4, 2, false, true>;
using CfgF8128 = GemmCfg<128, 128, 2, 2, false, true>;
using CfgNN256 = GemmCfg<256, 256, 4, 2, true>;
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

// Tile choice (measured on MI355X at the Wan shapes): the 8-wave 256x256 tile
// whenever it still gives every CU a tile; the 4-wave 128x128 tile otherwise.
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

extern "C" int mlora_gemm_fwd_fp8(const void *xq, int64_t ldx, const float *x_scale, int64_t M, int64_t K,
                                  const void *wq, int64_t ldw, const float *w_scale, int64_t N, const void *bias,
                                  int bias_dtype, const void *h_rows, int64_t ldh, const void *const *b_ptrs,
                                  const int32_t *ranks, int32_t n_adapters, const int64_t *seg_offsets,
                                  const int32_t *adapter_ids, int32_t n_segments, void *y, int64_t ldy, int accumulate,
                                  void *stream) {
  GemmArgs a{};
  int st = fill_common(a, M, K, N, h_rows, ldh, b_ptrs, ranks, n_adapters, seg_offsets, adapter_ids, n_segments);
  if (st) return st;
  if ((st = check_fp8_matrix(xq, ldx, M, K))) return st;
  if ((st = check_fp8_matrix(wq, ldw, N, K))) return st;
  if ((st = check_bf16_matrix(y, ldy, M, N))) return st;
  if (M == 0 || N == 0) return MLORA_OK;
  if (y == nullptr || xq == nullptr || wq == nullptr || x_scale == nullptr || w_scale == nullptr) return MLORA_ERR_INVALID;
  if (K == 0) return MLORA_ERR_UNSUPPORTED;  // the contraction loop starts with an e4m3 k-tile
  if (!aligned16(w_scale)) return MLORA_ERR_UNSUPPORTED;
  if (bias != nullptr) {
    if (bias_dtype != MLORA_F32 && bias_dtype != MLORA_BF16) return MLORA_ERR_UNSUPPORTED;
    if (!aligned16(bias)) return MLORA_ERR_UNSUPPORTED;
  }
  if (ldx * 256 >= (int64_t)kOOB || ldw * 256 >= (int64_t)kOOB || !offsets_fit(ldy, 256)) return MLORA_ERR_LIMIT;
  a.P = xq;
  a.Q = wq;
  a.psc = x_scale;
  a.qsc = w_scale;
  a.ldp = ldx;
  a.ldq = ldw;
  a.bias = bias;
  a.bias_dtype = bias ? bias_dtype : -1;
  a.Y = static_cast<uint16_t *>(y);
  a.ldy = ldy;
  a.accumulate = accumulate ? 1 : 0;
  return dispatch_gemm<CfgF8256, CfgF8128>(a, static_cast<hipStream_t>(stream));
}
