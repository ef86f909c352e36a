// Base-projection GEMMs of the multi-LoRA linear, with the LoRA term fused in.
//
//   forward : Y[m,n]  = bf16( Σ_k X[m,k]·W[n,k]  + bias[n] + Σ_j Hs[m,j]·B_a[n,j] )
//   dX      : dX[m,k] = bf16( Σ_n dY[m,n]·W[n,k]            + Σ_j Gs[m,j]·A_a[j,k] )
//
// Both are C = P·Q with P row-major [M, Kc] (contraction contiguous) and Q
// either "NT" ([Ncols, Kc], contraction contiguous: W in the forward, B_a) or
// "NN" ([Kc, Ncols]: W and A_a in dX). The LoRA term is more contraction: after
// the main loop over Kc, every segment that overlaps the tile's rows and has
// an adapter runs ceil(r/32) extra k-tiles with P = Hs rows of that segment
// (other rows read as zero) and Q = that adapter's B_a / A_a. Y is written once.
//
// gfx950 mapping: v_mfma_f32_32x32x16_bf16, wave64. A workgroup of WM x WN
// waves owns a BM x BN tile; each wave a (BM/WM) x (BN/WN) sub-tile whose fp32
// accumulators stay in registers. Operand k-tiles of 32 contraction elements
// stream through a ring of LDS stages filled by direct-to-LDS loads issued
// one by one between the MFMAs, STAGES-1 k-tiles ahead (one barrier per
// k-tile); the 256x256 NT tile instead alternates MFMA-only and load/read
// phases between the two waves of each SIMD (contract_tile_pp). Global reads use raw buffer
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
  const float *qsc;    // fp8 forward: per-row scale of Q [Ncols] (nullptr: 1)
  const void *bias;
  uint16_t *Y;
  int64_t ldp, ldq, lde, ldy;
  int32_t M, Ncols, Kc;
  int32_t bias_dtype;  // -1: none
  int32_t accumulate;
  int32_t tiles_m, tiles_n;
  int32_t group_m;  // row tiles per group of the tile order (set by launch_gemm)
  // >= 0: this launch runs 128x128 quarters of the 256x256 tiles tail_base, tail_base + 1, ... of
  // the tile order of a tiles_m x tiles_n grid of 256x256 tiles (four workgroups per tile);
  // -1: one workgroup per tile of its own size (set by launch_gemm)
  int32_t tail_base;
  AdapterTable ext;  // NT: B_a [Ncols, r]; NN: A_a [r, Ncols]
  SegTable seg;
  // Gated residual epilogue (gemm_kernel<C, true>): the stored value is
  // bf16(res[m, n] + bf16(Y[m, n])·gate[m / gate_rows, n]) instead of Y; with res_f32 the
  // residual stream is float32: Yf[m, n] = res[m, n] + bf16(Y[m, n])·gate (fp32 out).
  const void *res;
  const float *gate;
  float *Yf;
  int64_t ldres, ldgate;
  int32_t gate_rows;
  int32_t res_f32;
  // Stacked linears (gemm_kernel<C, RESID, STK>), G = groups of them.
  // STK 1 (forward): the output columns hold the G linears side by side, group_cols columns each
  // (a multiple of the tile width), linear g's columns stored to Yg[g] (its own [M, group_cols]
  // matrix, pitch ldy); a tile of linear g takes its LoRA rows from E's columns
  // [g·group_ecols, g·group_ecols + r).
  // STK 2 (dX): the main contraction runs over the G linears' dY in turn, group_cols columns each:
  // P = Pg[g] (pitch ldp) against Q's contraction columns [g·group_cols, (g+1)·group_cols).
  int32_t groups, group_cols, group_ecols;
  uint16_t *Yg[MLORA_MAX_STACKED];
  const uint16_t *Pg[MLORA_MAX_STACKED];
};

template <int BM_, int BN_, int WM_, int WN_, bool NN_, bool F8_ = false, int KB_ = 128, int STAGES_ = 2,
          bool RING5_ = false, bool SPREAD_ = false, bool PP_ = false>
struct GemmCfg {
  static constexpr int BM = BM_, BN = BN_, WM = WM_, WN = WN_;
  static constexpr bool NN = NN_;
  static constexpr bool F8 = F8_;  // main contraction in e4m3 (v_mfma_scale_f32_32x32x64_f8f6f4)
  static_assert(!(NN && F8), "the fp8 main contraction is NT only");
  static constexpr int NW = WM * WN;
  static constexpr int THREADS = 64 * NW;
  static constexpr int TM = BM / WM / 32;  // 32x32 MFMA tiles per wave along m
  static constexpr int TN = BN / WN / 32;  // ... along n
  // A k-tile holds KB bytes of contraction per row (KB / 2 bf16 or KB e4m3) as
  // CPR chunks of 16 bytes; an NN Q k-tile holds KB / 2 natural rows of BN
  // columns. 128-byte rows make every direct-to-LDS load read whole 128-byte
  // lines (64-byte rows move ~40% fewer bytes per CU, measured).
  static constexpr int KB = KB_;
  static_assert(KB == 64 || KB == 128, "64- or 128-byte k-tile rows");
  static constexpr int CPR = KB / 16;    // chunks per row
  static constexpr int RPD = 1024 / KB;  // rows per 1 KB load
  static constexpr int NSUB = KB / 32;   // 16-deep bf16 substeps per k-tile (an e4m3 substep takes two)
  static_assert(NSUB % 2 == 0, "the step's last substep reads the next tile's first into the first buffer");
  static constexpr int STAGES = STAGES_;  // LDS ring depth
  static constexpr int A_BYTES = BM * KB, B_BYTES = BN * KB;  // one stage of P / of Q
  static constexpr int A_DMA = A_BYTES / 1024 / NW;           // 1 KB direct-to-LDS loads per wave for the P tile
  static constexpr int B_DMA = B_BYTES / 1024 / NW;           // the same for the Q tile
  static constexpr int QROW = BN * 2;                         // NN: bytes per contraction row
  static constexpr int QCPR = BN / 8;                         // NN: 16-byte chunks per row
  static constexpr int QRPD = 1024 / QROW;                    // NN: rows per 1 KB load
  static_assert(A_DMA * NW * 1024 == A_BYTES && B_DMA * NW * 1024 == B_BYTES, "tiles split into 1 KB loads per wave");
  static_assert(!NN || (QCPR >= 16 && QRPD >= 1), "NN rows hold at least 16 chunks");
  static constexpr int NDMA = A_DMA + B_DMA;  // 1 KB loads per wave and k-tile
  static constexpr int TMN = TM * TN;  // MFMAs per wave and 16-deep bf16 substep (or e4m3 substep)
  // LDS layout. Stages: P stages 0..STAGES-1 | Q stages 0..STAGES-1; k-tile t
  // in stage t % STAGES, and a step loads the k-tile STAGES ahead into the
  // stage its barrier freed. RING5 (bf16 256x256, 128-byte rows): five 32 KB
  // slots, k-tile t's P in slot 2t % 5 and Q in slot (2t + 1) % 5: a step
  // loads the k-tile 2 ahead, its P into the slot the previous barrier freed
  // (issued before the barrier: in the first substep, or over all of them with
  // SPREAD) and its Q into the slot its own barrier frees — 1.5 k-tiles in
  // flight instead of 1 in the same 160 KB.
  static constexpr bool RING5 = RING5_;
  static_assert(!RING5 || (A_BYTES == 32768 && B_BYTES == 32768), "slots hold one 256-row operand tile");
  static constexpr int PERIOD = RING5 ? 5 : STAGES;  // steps until the LDS offsets repeat
  static constexpr int AHEAD = RING5 ? 2 : STAGES;   // a step loads the k-tile this far ahead
  static constexpr int B_BASE = RING5 ? 0 : STAGES * A_BYTES;
  static constexpr int LDS_BYTES = RING5 ? 5 * A_BYTES : STAGES * (A_BYTES + B_BYTES);
  // LDS offsets of the P and Q tiles of a k-tile in phase ph (its index mod
  // PERIOD). Stages: the Q fragment addresses carry B_BASE, so q_off is
  // relative to it and stays within the 16-bit ds_read offset field.
  // SPREAD (RING5): the P-half loads a step issues before its barrier are
  // spread over all the substeps before the barrier instead of the first one
  // (fewer loads queued at the texture unit at once: 1-3% per launch).
  static constexpr bool SPREAD = SPREAD_;
  // PP: the ping-pong schedule of contract_tile_pp (8-wave 256x256 bf16 NT tiles; its own LDS ring)
  static constexpr bool PP = PP_;
  static_assert(!PP || (RING5 && !F8 && !NN && NW == 8), "the ping-pong schedule runs 8-wave bf16 NT tiles on the 5-slot ring");
  static constexpr int p_off(int ph) { return RING5 ? ((2 * ph) % 5) * A_BYTES : ph * A_BYTES; }
  static constexpr int q_off(int ph) { return RING5 ? ((2 * ph + 1) % 5) * A_BYTES : ph * B_BYTES; }
  static_assert(LDS_BYTES <= 163840, "the ring must fit the 160 KB of LDS");
  // occupancy the register budget is sized for: a 256x256 tile fills the LDS
  // (one workgroup per CU, NW / 4 waves per SIMD); 128x128 tiles run two
  // workgroups per CU
  static constexpr int WAVES_PER_SIMD = BM == 256 ? (NW >= 8 ? NW / 4 : 1) : 2;
};

// Chunk swizzle of a tile row with CPR chunks: chunk c of row r sits at slot
// c ^ swzk<CPR>(r). The 16 lanes of one fragment read (16 consecutive
// 16-aligned rows, one chunk) then hit 16 distinct 16-byte bank groups of the
// 256-byte bank period: 8 chunks per row — the slot carries r % 8, the parity
// of r / 8 picks the half period; 4 chunks — the row sits at r % 4 of the
// period, the slot carries (r / 4) % 4. Both depend on r % 16 only.
template <int CPR>
__device__ __forceinline__ int swzk(int row) {
  if constexpr (CPR == 8) return swz(row);
  else return (row >> 2) & 3;
}

// One contraction source (wave-uniform): P rows valid in [row_lo, row_hi),
// contraction valid below klim (elements) for both operands. esz is the
// element size (2: bf16, 1: e4m3); an LDS k-tile always holds KB bytes of
// contraction per row, i.e. KB / esz elements.
struct KSource {
  const char *P;
  const char *Q;
  int64_t ldp_b, ldq_b;  // row pitches in bytes
  int32_t row_lo, row_hi;
  int32_t klim;
  int32_t esz;
};

// Per-thread state of one contraction source. Global tiles go to LDS with the
// gfx950 direct-to-LDS buffer load: one wave instruction fills 1 KB (RPD rows
// of CPR chunks); lane L lands at chunk slot L % CPR of row L / CPR of that KB,
// so it fetches logical chunk (L % CPR) ^ swzk(row). The swizzle depends on
// row % 16 only, so the 1 KB loads of a wave differ by a whole number of rows
// plus (8-row loads) one of two lane patterns, even or odd load; the load's row
// and the tile's k offset travel in soffset.
template <class C>
struct Pipe {
  __amdgpu_buffer_rsrc_t rp, rq;
  int32_t a_off[2];  // this lane's P chunk offset at k = 0 in an even / odd load (rows past the tile: kOOB)
  int32_t a_kc[2];   // contraction index of that chunk
  int32_t a_row0;    // first P row (tile-local) of this wave's loads
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
    a_row0 = C::RPD * wave * C::A_DMA;
#pragma unroll
    for (int par = 0; par < 2; ++par) {
      const int c = (lane % C::CPR) ^ swzk<C::CPR>(C::RPD * par + lane / C::CPR);
      a_kc[par] = chunk_elems * c;
      a_off[par] = (lane / C::CPR) * ldp_b + 16 * c;
    }
    if constexpr (!C::NN) {
      rq = make_rsrc(s.Q + (int64_t)n0 * s.ldq_b, (int64_t)(Ncols - n0) * s.ldq_b);
      b_row0 = C::RPD * wave * C::B_DMA;
#pragma unroll
      for (int par = 0; par < 2; ++par) {
        const int c = (lane % C::CPR) ^ swzk<C::CPR>(C::RPD * par + lane / C::CPR);
        b_kc[par] = chunk_elems * c;
        b_off[par] = (lane / C::CPR) * ldq_b + 16 * c;  // rows past Ncols fall outside rq
      }
    } else {
      // NN (bf16 only): rows are contraction indices, chunk c of row k at slot c ^ (4 * (k & 3))
      rq = make_rsrc(s.Q + 2 * n0, (int64_t)s.klim * s.ldq_b);
      const int p = lane % C::QCPR, rl = lane / C::QCPR;
#pragma unroll
      for (int par = 0; par < 2; ++par) {
        const int cc = p ^ (4 * ((C::QRPD * par + rl) & 3));
        b_off[par] = (n0 + 8 * cc < Ncols) ? rl * ldq_b + 16 * cc : kOOB;
      }
      b_kc[0] = b_kc[1] = rl;  // row of this lane within its 1 KB load
    }
  }

  // Issue 1 KB load number q (of NDMA per wave) of the k-tile starting at k0
  // into the LDS tiles of phase ph: q < A_DMA are P rows, the rest Q.
  // live == false turns every lane's offset out of range: the instruction then
  // moves no data.
  __device__ __forceinline__ void issue_one(MLORA_LDS char *lds, int q, int ph, int k0, int wave, int lane, bool KMASK,
                                            bool live) const {
    if (q < C::A_DMA) {
      const int blk = wave * C::A_DMA + q;  // wave-uniform
      MLORA_LDS void *dst = lds + C::p_off(ph) + blk * 1024;
      const int row = a_row0 + C::RPD * q;
      const int par = blk & 1;
      int32_t off = a_off[par];
      if (p_rows > 0 && row + lane / C::CPR < p_rows) off = kOOB;  // rows of an earlier segment
      if (KMASK && k0 + a_kc[par] >= klim) off = kOOB;
      if (!live) off = kOOB;
      const int32_t soff = row * ldp_b + k0 * esz;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rp, dst, 16, off, soff, 0, 0);
    } else if constexpr (!C::NN) {
      const int qb = q - C::A_DMA;
      const int blk = wave * C::B_DMA + qb;
      MLORA_LDS void *dst = lds + C::B_BASE + C::q_off(ph) + blk * 1024;
      const int row = b_row0 + C::RPD * qb;
      const int par = blk & 1;
      int32_t off = (KMASK && k0 + b_kc[par] >= klim) ? kOOB : b_off[par];
      if (!live) off = kOOB;
      const int32_t soff = row * ldq_b + k0 * esz;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rq, dst, 16, off, soff, 0, 0);
    } else {
      const int blk = wave * C::B_DMA + (q - C::A_DMA);  // wave-uniform
      MLORA_LDS void *dst = lds + C::B_BASE + C::q_off(ph) + blk * 1024;
      const int row = C::QRPD * blk;
      int32_t off = (KMASK && k0 + row + b_kc[0] >= klim) ? kOOB : b_off[blk & 1];
      if (!live) off = kOOB;
      const int32_t soff = (k0 + row) * ldq_b;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rq, dst, 16, off, soff, 0, 0);
    }
  }
};

// Byte addresses (first 32-row tile, phase 0 layout: P at 0, Q at B_BASE) of
// this lane's fragments for each 16-deep substep of a k-tile; further tiles
// are +32 * KB bytes and the phase's p_off / q_off is added as a constant.
// NN: b[j] is the first of the two transposing reads of tile j at substep 0
// (substep h adds 16 rows, the second read 4 rows). ds_read_b64_tr_b16 gives
// lane j of a 16-lane group element e = element (j & 3) of the 8 bytes
// addressed by lane 4e + (j >> 2); lane i pointing at row k0 + (i >> 2),
// column c0 + 4(i & 3) therefore yields 4 consecutive contraction values of
// column c0 + j: half of the B fragment of v_mfma_f32_32x32x16_bf16.
// LDS offsets past 64 KB do not fit the 16-bit offset field of a ds_read, so
// each fragment address also has copies 64 KB and 128 KB higher (a1/a2,
// b1/b2) that the compiler cannot see through: reads of the upper slots use
// them with an in-range immediate instead of one hoisted address register per
// (substep, tile, slot).
__device__ __forceinline__ int32_t opaque_vgpr(int32_t x) {
  asm volatile("" : "+v"(x));
  return x;
}
// The same for a wave-uniform value: computed from where it is used (no hoisted copies).
__device__ __forceinline__ int32_t opaque_sgpr(int32_t x) {
  asm volatile("" : "+s"(x));
  return x;
}

template <class C>
struct FragAddr {
  int32_t a[C::NSUB], b[C::NN ? C::TN : C::NSUB];
  int32_t a1[C::NSUB], a2[C::NSUB], b1[C::NSUB], b2[C::NSUB];
  __device__ __forceinline__ void init(int wm0, int wn0, int lane) {
    const int z = swzk<C::CPR>(lane & 31);  // lane-constant: fragment rows are 32-aligned + lane
#pragma unroll
    for (int h = 0; h < C::NSUB; ++h) {
      const int slot = (2 * h + (lane >> 5)) ^ z;
      a[h] = (wm0 + (lane & 31)) * C::KB + 16 * slot;
      if constexpr (!C::NN) b[h] = C::B_BASE + (wn0 + (lane & 31)) * C::KB + 16 * slot;
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
#pragma unroll
    for (int h = 0; h < C::NSUB; ++h) {
      a1[h] = opaque_vgpr(a[h] + 65536);
      a2[h] = opaque_vgpr(a[h] + 131072);
      if constexpr (!C::NN) {
        b1[h] = opaque_vgpr(b[h] + 65536);
        b2[h] = opaque_vgpr(b[h] + 131072);
      }
    }
  }
};

// A lane's operand fragments of one 16-deep substep of a k-tile: the chunk of
// every 32-row tile of P (a) and of Q (b). A bf16 k-tile multiplies substep h
// on its own; an e4m3 substep multiplies two of them at once as the 32-byte
// fragments of v_mfma_scale_f32_32x32x64_f8f6f4, whose lane l holds 32
// contraction bytes of row (A) / column (B) l % 32 at positions
// 32 * (l / 32) + e; any assignment of contraction indices to (l / 32, e) gives
// the same product as long as A and B agree, so the fp8 form reads exactly
// the bytes of the bf16 form.
template <class C>
struct Half {
  u32x4 a[C::TM];
  u32x4 b[C::TN];
};

// LDS reads per substep visible to the compiler: the P chunks, then (NT) the
// Q chunks; NN Q chunks come from read_q_nn (assembly).
template <class C>
constexpr int half_reads() {
  return C::NN ? C::TM : C::TM + C::TN;
}

// Read number r of substep h of the k-tile in phase PH.
template <class C, int PH>
__device__ __forceinline__ void read_frag(int r, int h, Half<C> &f, const MLORA_LDS char *lds, const FragAddr<C> &fa) {
  if (r < C::TM) {
    const int off = 32 * C::KB * r + C::p_off(PH);
    const int32_t base = off >= 131072 ? fa.a2[h] : off >= 65536 ? fa.a1[h] : fa.a[h];
    f.a[r] = *(const lds_u4 *)(lds + base + (off & 65535));
    return;
  }
  if constexpr (!C::NN) {
    const int j = r - C::TM;
    const int off = 32 * C::KB * j + C::q_off(PH);
    const int32_t base = off >= 131072 ? fa.b2[h] : off >= 65536 ? fa.b1[h] : fa.b[h];
    f.b[j] = *(const lds_u4 *)(lds + base + (off & 65535));
  }
}

// NN: all TN Q fragments of substep h of the k-tile in phase PH: pairs of
// transposing reads (rows 16h + 8(l/32) + (l%16)/4 and 4 rows further) in one
// block that also waits for them (see lds_read_tr16_x4).
template <class C, int PH>
__device__ __forceinline__ void read_q_nn(Half<C> &f, const MLORA_LDS char *lds, const FragAddr<C> &fa, int h) {
  const MLORA_LDS char *base = lds + (C::q_off(PH) + 16 * C::QROW * h);
  lds_read_tr16<C::TN, 4 * C::QROW>(base, fa.b, f.b);
}

// Substep h of the k-tile in phase PH, all reads back to back.
template <class C, int PH>
__device__ __forceinline__ void read_half(Half<C> &f, int h, const MLORA_LDS char *lds, const FragAddr<C> &fa) {
#pragma unroll
  for (int r = 0; r < half_reads<C>(); ++r) read_frag<C, PH>(r, h, f, lds, fa);
  if constexpr (C::NN) read_q_nn<C, PH>(f, lds, fa, h);
}

// One bf16 substep: TMN MFMAs on the fragments in `x` while substep rh of the
// k-tile in phase RS is read into rd and loads Q0..Q1-1 of the k-tile at k0
// go to the LDS tiles of phase LS. Reads and loads are spread evenly over the MFMAs
// (scheduling hints keep that order): issued back to back, loads fill the
// texture unit's queue and stall the wave's MFMA issue behind them. MFMA rows
// <- Q (n), columns <- P (m), so each lane ends up with 4 consecutive n of
// one row m, stored as one 8-byte write.
template <class C, int RS, int LS, int Q0, int Q1>
__device__ __forceinline__ void mma_half(f32x16 (&acc)[C::TM][C::TN], const Half<C> &x, Half<C> &rd, int rh,
                                         MLORA_LDS char *lds, const FragAddr<C> &fa, const Pipe<C> &pipe, int k0,
                                         bool kmask, bool live, int wave, int lane) {
  constexpr int NM = C::TMN;
  constexpr int NR = half_reads<C>();
  constexpr int NQ = Q1 - Q0;  // loads q = Q0 + (g * NQ) / NM ... follow MFMA g
#pragma unroll
  for (int g = 0; g < NM; ++g) {
#pragma unroll
    for (int r = (g * NR) / NM; r < ((g + 1) * NR) / NM; ++r) read_frag<C, RS>(r, rh, rd, lds, fa);
    if constexpr (C::NN) {
      if (g == NM / 2) read_q_nn<C, RS>(rd, lds, fa, rh);
    }
    const int j = g / C::TM, i = g % C::TM;
    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(as_bf16x8(x.b[j]), as_bf16x8(x.a[i]), acc[i][j], 0, 0, 0);
#pragma unroll
    for (int q = (g * NQ) / NM; q < ((g + 1) * NQ) / NM; ++q)
      pipe.issue_one(lds, Q0 + q, LS, k0, wave, lane, kmask, live);
  }
#pragma unroll
  for (int g = 0; g < NM; ++g) {
    const int nr = ((g + 1) * NR) / NM - (g * NR) / NM;
    const int nq = ((g + 1) * NQ) / NM - (g * NQ) / NM;
#pragma unroll
    for (int r = 0; r < nr; ++r) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // one DS read
    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);                                // one MFMA
#pragma unroll
    for (int q = 0; q < nq; ++q) __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);  // one load
  }
}

// The fragments of one e4m3 substep: two 16-byte chunks of each 32-row tile
// as one 32-byte MFMA operand (bf16 substep 2u in elements 0-3, 2u+1 in 4-7).
typedef int i32x8 __attribute__((ext_vector_type(8)));
template <class C>
struct Frag8 {
  i32x8 a[C::TM];
  i32x8 b[C::TN];
};

// Read number r (P tiles, then Q tiles) of e4m3 substep u of the k-tile in phase RS.
template <class C, int RS>
__device__ __forceinline__ i32x8 read_frag8(int r, int u, const MLORA_LDS char *lds, const FragAddr<C> &fa) {
  Half<C> lo, hi;
  read_frag<C, RS>(r, 2 * u, lo, lds, fa);
  read_frag<C, RS>(r, 2 * u + 1, hi, lds, fa);
  const u32x4 l = r < C::TM ? lo.a[r] : lo.b[r - C::TM];
  const u32x4 h = r < C::TM ? hi.a[r] : hi.b[r - C::TM];
  return i32x8{(int)l[0], (int)l[1], (int)l[2], (int)l[3], (int)h[0], (int)h[1], (int)h[2], (int)h[3]};
}

// One e4m3 substep (NT only): TMN scaled MFMAs on the fragments in f, column
// by column; once column j's MFMAs are issued its Q fragment is replaced by
// that of e4m3 substep RU of the k-tile in phase RS, and the P fragments after
// the last column, so the next substep's fragments reuse the registers. Loads
// Q0..Q1-1 of the k-tile at k0 go to the tiles of phase LS, spread over the MFMAs.
template <class C, int RS, int RU, int LS, int Q0, int Q1>
__device__ __forceinline__ void mma_fp8(f32x16 (&acc)[C::TM][C::TN], Frag8<C> &f, MLORA_LDS char *lds,
                                        const FragAddr<C> &fa, const Pipe<C> &pipe, int k0, bool kmask, bool live,
                                        int wave, int lane) {
  static_assert(!C::NN, "e4m3 k-tiles are NT");
  constexpr int NM = C::TMN;
  constexpr int NQ = Q1 - Q0;  // loads q = Q0 + (g * NQ) / NM ... follow MFMA g
#pragma unroll
  for (int g = 0; g < NM; ++g) {
    const int j = g / C::TM, i = g % C::TM;
    acc[i][j] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(f.b[j], f.a[i], acc[i][j], 0, 0, 0, 127, 0, 127);
#pragma unroll
    for (int q = (g * NQ) / NM; q < ((g + 1) * NQ) / NM; ++q)
      pipe.issue_one(lds, Q0 + q, LS, k0, wave, lane, kmask, live);
    if (i == C::TM - 1) f.b[j] = read_frag8<C, RS>(C::TM + j, RU, lds, fa);
  }
#pragma unroll
  for (int i = 0; i < C::TM; ++i) f.a[i] = read_frag8<C, RS>(i, RU, lds, fa);
#pragma unroll
  for (int g = 0; g < NM; ++g) {
    const int nq = ((g + 1) * NQ) / NM - (g * NQ) / NM;
    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // one MFMA
#pragma unroll
    for (int q = 0; q < nq; ++q) __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);  // one load
    if (g % C::TM == C::TM - 1) __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);  // two DS reads
  }
  __builtin_amdgcn_sched_group_barrier(0x100, 2 * C::TM, 0);
}

// Finds the next LoRA source of this tile: the next segment from `seg` on that
// overlaps rows [m0, row_end) and has an adapter. Wave-uniform scalar code.
__device__ __forceinline__ bool next_lora_source(const GemmArgs &args, bool nn, int m0, int row_end, int &seg,
                                                 KSource &src, int ecol = 0) {
  while (seg < args.seg.n && args.seg.off[seg] < row_end) {
    const int a = args.seg.aid[seg];
    const int lo = max(args.seg.off[seg], m0), hi = min(args.seg.off[seg + 1], row_end);
    ++seg;
    if (a >= 0 && args.ext.rank[a] > 0 && lo < hi) {
      const int r = args.ext.rank[a];
      src = KSource{reinterpret_cast<const char *>(args.E + ecol), reinterpret_cast<const char *>(args.ext.ptr[a]),
                    2 * args.lde,
                    2 * (nn ? (int64_t)args.Ncols : (int64_t)r), lo, hi, r, 2};
      return true;
    }
  }
  return false;
}

// All contraction of one tile in a single pipelined loop over "virtual"
// k-tiles: first the main X·Wᵀ (or dY·W) tiles, then ceil(r / (KB/2)) tiles
// per LoRA segment overlapping the tile. At a source boundary the loader is
// re-pointed (a few scalars and two offsets); the LDS stages and the MFMA code
// are shared, so the accumulators stay in place. Tiles past a source's
// contraction length mask their chunks.
//
// Pipeline: k-tile t lives in the LDS tiles of phase t % PERIOD (see
// GemmCfg). Step t multiplies tile t substep by substep, each substep's
// fragments read during the previous one. Before its last substep every wave
// waits for its own loads of tile t+1 and the workgroup meets at a barrier:
// all of tile t+1 is then in LDS (the last substep reads its first fragments)
// and every wave has read all of tile t, whose tiles the loads of tile
// t+AHEAD now fill, spread over the MFMAs of the last substep (RING5: the P
// half of those loads goes, during the first substep, to the slot the
// previous barrier freed). Loads past the last tile are issued with every
// offset out of range (no data moves), so every step issues the same number
// of loads and the vmcnt thresholds are constants; the phase loop is unrolled
// so every LDS offset is a constant as well.
template <class C, int STK = 0>
__device__ __forceinline__ void contract_tile(f32x16 (&acc)[C::TM][C::TN], const GemmArgs &args, MLORA_LDS char *lds,
                                              const FragAddr<C> &fa, int m0, int n0, int tid) {
  constexpr int S = C::PERIOD, NSUB = C::NSUB, NDMA = C::NDMA;
  const int wave = wave_id(), lane = tid & 63;
  const int row_end = min(m0 + C::BM, args.M);
  // stacked forward: this tile's linear reads its own columns of the LoRA rows
  const int ecol = STK == 1 ? __builtin_amdgcn_readfirstlane((n0 / args.group_cols) * args.group_ecols) : 0;
  int grp = 0;  // stacked dX: the linear whose dY the main contraction is reading
  // the first segment that may overlap the tile: looked up when the LoRA sources start, so that
  // the scalar loads of the search do not delay the first k-tile loads
  int seg = -1;
  auto first_seg = [&]() {
    if (seg < 0) seg = args.E != nullptr ? seg_of_row(args.seg, m0) : args.seg.n;
  };
  Pipe<C> pipe;
  constexpr int esz0 = C::F8 ? 1 : 2;
  KSource src{static_cast<const char *>(args.P), static_cast<const char *>(args.Q), esz0 * args.ldp, esz0 * args.ldq,
              0, args.M, args.Kc, esz0};
  int bk = C::KB / src.esz;  // contraction elements per k-tile of the current source
  int ntile = (src.klim + bk - 1) / bk;
  // e4m3: the main contraction is padded to a multiple of S k-tiles (zero
  // chunks) so the bf16 LoRA k-tiles start at stage 0
  const int n_main = ntile;  // e4m3 k-tiles (F8), before the first LoRA tile
  if (ntile == 0) {
    first_seg();
    if (!next_lora_source(args, C::NN, m0, row_end, seg, src, ecol)) return;
    bk = C::KB / src.esz;
    ntile = (src.klim + bk - 1) / bk;
  }
  bool kmask = ntile * bk != src.klim;
  pipe.init(src, m0, n0, args.Ncols, tid);
  int t_in_src = 0;  // index of the tile being loaded within its source
  bool exhausted = false;
  int n_real = 1;  // k-tiles with data issued so far
  // moves the loader to the next k-tile; false once every source is done
  auto advance = [&]() -> bool {
    if (exhausted) return false;
    if (t_in_src + 1 < ntile) {
      ++t_in_src;
      ++n_real;
      return true;
    }
    if constexpr (STK == 2) {
      if (grp + 1 < args.groups) {  // the next linear's dY against its columns of Q
        ++grp;
        src = KSource{reinterpret_cast<const char *>(args.Pg[grp]),
                      reinterpret_cast<const char *>(args.Q) + 2 * (int64_t)grp * args.group_cols, 2 * args.ldp,
                      2 * args.ldq, 0, args.M, args.group_cols, 2};
        kmask = src.klim % bk != 0;
        pipe.init(src, m0, n0, args.Ncols, tid);
        t_in_src = 0;
        ++n_real;
        return true;
      }
    }
    first_seg();
    if (!next_lora_source(args, C::NN, m0, row_end, seg, src, ecol)) {
      exhausted = true;
      return false;
    }
    bk = C::KB / src.esz;
    ntile = (src.klim + bk - 1) / bk;
    kmask = src.klim % bk != 0;
    pipe.init(src, m0, n0, args.Ncols, tid);
    t_in_src = 0;
    ++n_real;
    return true;
  };
  static_for<C::AHEAD>([&](auto p) {  // the prologue loads k-tiles 0..AHEAD-1
    constexpr int P = decltype(p)::value;
    const bool live = P == 0 ? true : advance();
#pragma unroll
    for (int q = 0; q < NDMA; ++q) pipe.issue_one(lds, q, P, t_in_src * bk, wave, lane, kmask, live);
    return true;
  });
  wait_vmcnt<(C::AHEAD - 1) * NDMA>();  // this wave's loads of tile 0
  lds_pipeline_barrier();
  int t = 0;
  bool done = false;
  // Runs steps from tile t until every tile is done or t reaches stop_at; the
  // stage loop is unrolled so every LDS offset is a constant. e4m3: the bf16
  // LoRA k-tiles start where the e4m3 ones end, at phase t % S, so a partial
  // period runs first.
  auto run = [&](int stop_at, auto &&step) {
    if constexpr (C::F8) {
      const int p0 = t % S;
      if (p0 != 0 && !done && t < stop_at) static_for<S>([&](auto st) -> bool {
          if (decltype(st)::value < p0) return true;
          step(st);
          ++t;
          done = t >= n_real;
          return !done && t < stop_at;
        });
    }
    while (!done && t < stop_at) static_for<S>([&](auto st) -> bool {
        step(st);
        ++t;
        done = t >= n_real;
        return !done && t < stop_at;
      });
  };
  // this wave's loads still allowed in flight at the barrier of a step: those
  // of the tiles after t+1 (RING5: the P half of tile t+2, issued before the
  // barrier)
  constexpr int PQ = C::RING5 ? C::A_DMA : 0;  // loads of a step issued before its barrier
  constexpr int WAIT = C::RING5 ? PQ : (C::AHEAD - 2) * NDMA;
  Half<C> h0, h1;  // fragments of the current and the next substep
  if constexpr (C::F8) {
    // e4m3 steps (NSUB / 2 substeps of TMN scaled MFMAs), the same barrier
    // and load placement as the bf16 steps (RING5: the P half of tile t+2 in
    // the substeps before the barrier, the Q half after it).
    constexpr int NS8 = NSUB / 2;
    Frag8<C> f;
#pragma unroll
    for (int r = 0; r < C::TM; ++r) f.a[r] = read_frag8<C, 0>(r, 0, lds, fa);
#pragma unroll
    for (int r = 0; r < C::TN; ++r) f.b[r] = read_frag8<C, 0>(C::TM + r, 0, lds, fa);
    run(n_main, [&](auto st) {
      constexpr int ST = decltype(st)::value, NS = (ST + 1) % S, LS = (ST + C::AHEAD) % S;
      const bool live = advance();
      const int k0 = t_in_src * bk;
      static_for<NS8>([&](auto u_c) {
        constexpr int U = decltype(u_c)::value;
        if constexpr (U == NS8 - 1) {
          wait_vmcnt<WAIT>();  // this wave's loads of tile t + 1
          lds_pipeline_barrier();
          mma_fp8<C, NS, 0, LS, PQ, NDMA>(acc, f, lds, fa, pipe, k0, kmask, live, wave, lane);
        } else {
          constexpr int Q0 = U * PQ / (NS8 - 1), Q1 = (U + 1) * PQ / (NS8 - 1);
          mma_fp8<C, ST, U + 1, LS, Q0, Q1>(acc, f, lds, fa, pipe, k0, kmask, live, wave, lane);
        }
        return true;
      });
    });
#pragma unroll
    for (int r = 0; r < C::TM; ++r)
      h0.a[r] = u32x4{(uint32_t)f.a[r][0], (uint32_t)f.a[r][1], (uint32_t)f.a[r][2], (uint32_t)f.a[r][3]};
#pragma unroll
    for (int r = 0; r < C::TN; ++r)
      h0.b[r] = u32x4{(uint32_t)f.b[r][0], (uint32_t)f.b[r][1], (uint32_t)f.b[r][2], (uint32_t)f.b[r][3]};
  } else {
    read_half<C, 0>(h0, 0, lds, fa);
  }
  // bf16 steps: substep s from h[s % 2] while substep s+1 is read into the
  // other; before the last substep the wait and barrier; the last substep
  // reads substep 0 of tile t+1.
  run(INT32_MAX, [&](auto st) {
    constexpr int ST = decltype(st)::value, NS = (ST + 1) % S, LS = (ST + C::AHEAD) % S;
    const bool live = advance();  // tile t + AHEAD
    const int k0 = t_in_src * bk;
    static_for<NSUB>([&](auto s_c) {
      constexpr int SS = decltype(s_c)::value;
      Half<C> &x = SS % 2 == 0 ? h0 : h1;
      Half<C> &y = SS % 2 == 0 ? h1 : h0;
      if constexpr (SS < NSUB - 1) {
        constexpr int Q0 = C::SPREAD ? SS * PQ / (NSUB - 1) : 0;
        constexpr int Q1 = C::SPREAD ? (SS + 1) * PQ / (NSUB - 1) : (SS == 0 ? PQ : 0);
        mma_half<C, ST, LS, Q0, Q1>(acc, x, y, SS + 1, lds, fa, pipe, k0, kmask, live, wave, lane);
      } else {
        wait_vmcnt<WAIT>();  // this wave's loads of tile t + 1
        lds_pipeline_barrier();
        mma_half<C, NS, LS, PQ, NDMA>(acc, x, y, 0, lds, fa, pipe, k0, kmask, live, wave, lane);
      }
      return true;
    });
  });
  wait_vmcnt<0>();
}

// Direct-to-LDS loads of one operand for the ping-pong schedule (contract_tile_pp, NT tiles). An
// operand k-tile of 32 KB is 32 blocks of 1 KB: block blk holds rows RPD·blk .. RPD·blk + RPD - 1
// of P or Q; the lane layout and swizzle are those of Pipe. Every source is bf16 here.
template <class C>
struct PPLoad {
  __amdgpu_buffer_rsrc_t r;
  int32_t off[2];  // this lane's offset in an even / odd block at k = 0 (kOOB: past the operand)
  int32_t ld_b, klim;
  int32_t p_rows;  // P: tile rows below this index belong to an earlier segment (read as zero)

  // the logical chunk this lane fetches in an even / odd block (the swizzle of Pipe)
  static __device__ __forceinline__ int chunk(int par, int lane) {
    return (lane % C::CPR) ^ swzk<C::CPR>(C::RPD * par + lane / C::CPR);
  }
  __device__ __forceinline__ void init_rows(const char *base, int64_t ldb, int64_t rows, int32_t masked, int32_t kl,
                                            int lane) {
    klim = kl;
    ld_b = (int32_t)ldb;
    p_rows = masked;
    r = make_rsrc(base, rows * ldb);
#pragma unroll
    for (int par = 0; par < 2; ++par) off[par] = (lane / C::CPR) * ld_b + 16 * chunk(par, lane);
  }
  // P: rows [row_lo, row_hi) of the tile at m0
  __device__ __forceinline__ void init_p(const KSource &s, int m0, int lane) {
    init_rows(s.P + (int64_t)m0 * s.ldp_b, s.ldp_b, s.row_hi - m0, max(s.row_lo, m0) - m0, s.klim, lane);
  }
  // Q: the Ncols - n0 rows from n0
  __device__ __forceinline__ void init_q(const KSource &s, int n0, int Ncols, int lane) {
    init_rows(s.Q + (int64_t)n0 * s.ldq_b, s.ldq_b, Ncols - n0, 0, s.klim, lane);
  }
  // Whether a k-tile needs the masks of issue (wave-uniform): rows of an earlier segment, a
  // partial last k-tile, or a tile past the last one. Every main-contraction tile of a whole
  // number of k-tiles needs none.
  __device__ __forceinline__ bool masked(bool kmask, bool live) const { return p_rows > 0 || kmask || !live; }
  // Block blk of the k-tile at k0 to LDS address dst. live == false turns every lane's offset
  // out of range: no data moves. MASK: apply the masks (see masked). Lane-derived values other
  // than the offsets are recomputed here (VALU is idle in the phases that issue loads) instead of
  // being held in registers across the k-loop.
  template <bool MASK>
  __device__ __forceinline__ void issue(MLORA_LDS char *dst, int blk, int k0, bool kmask, bool live, int lane) const {
    int32_t o = off[blk & 1];
    const int row = C::RPD * blk;
    if constexpr (MASK) {
      if (p_rows > 0 && row + lane / C::CPR < p_rows) o = kOOB;  // rows of an earlier segment
      if (kmask && k0 + 8 * chunk(blk & 1, lane) >= klim) o = kOOB;
      if (!live) o = kOOB;
    }
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, dst, 16, o, row * ld_b + 2 * k0, 0, 0);
  }
};

// A barrier between two phases of the ping-pong schedule; nothing is scheduled across it.
__device__ __forceinline__ void phase_barrier() {
  __builtin_amdgcn_sched_barrier(0);
  lds_pipeline_barrier();
  __builtin_amdgcn_sched_barrier(0);
}

// The contraction of one 256x256 bf16 tile (8 waves, 64x128 each) in a ping-pong schedule. Waves
// 0-3 (X) and 4-7 (Y) share the SIMDs pairwise (wave w with w + 4) and alternate phases: while
// one wave of a SIMD multiplies a whole k-tile from registers (32 MFMAs, no other instruction),
// the other issues its loads and reads all of its fragments of a k-tile from LDS; every phase
// ends at a workgroup barrier. So the MFMA pipe of each SIMD is fed by one wave at a time,
// without the fragment reads' waits or the loads' issue between its MFMAs.
//
// LDS: three Q slots of 32 KB (k-tile t's Q in slot t % 3), and P in 128-row halves, two slots
// of 16 KB for the top halves and two for the bottom ones (t % 2): X computes rows 0-127 and
// reads only the top halves, Y rows 128-255 and the bottom ones. Phase 2t: X reads k-tile t and
// issues Q(t+2) blocks 0-15 and Pbot(t+1); phase 2t+1: Y reads k-tile t and issues Q(t+2)
// blocks 16-31 and Ptop(t+2). Each load goes to the slot of k-tile t-1 (Q, Pbot) or t (Ptop),
// whose last reads were in the phase before. Every wave waits for its previous phase's loads at
// the end of each of its read phases (vmcnt(8)): a load has three phases to land.
//
// The last step drains every wave's loads before the last barrier; after it X stages its rows
// while Y still multiplies, so the epilogue (store_staged) needs no workgroup barrier.
//
// The k-tiles are contract_tile's sequence (the main contraction, then the LoRA tiles), walked
// by both sides; X's P loads trail its walk by one k-tile. Each accumulator takes its MFMAs in
// the same k order as in contract_tile, so the results are the same bit for bit.
template <class C, int STK = 0>
__device__ __forceinline__ void contract_tile_pp(f32x16 (&acc)[C::TM][C::TN], const GemmArgs &args,
                                                 MLORA_LDS char *lds, int wm0, int wn0, int m0, int n0, int tid) {
  static_assert(C::RING5 && !C::F8 && !C::NN && C::NW == 8 && C::NSUB == 4 && C::KB == 128,
                "8-wave 256x256 bf16 NT tiles of 128-byte k-tile rows");
  constexpr int QB = 0, PT = 3 * 32768, PB = PT + 2 * 16384;  // Q slots, P-top and P-bottom half slots
  constexpr int PER = 6;                                      // steps until the slots repeat
  static_assert(PB + 2 * 16384 <= C::LDS_BYTES, "the ring fits the LDS");
  constexpr int NSUB = C::NSUB;
  const int wave = wave_id(), lane = tid & 63;
  const bool xside = wave < 4;
  const int lw = wave & 3;
  const int qblk0 = (xside ? 0 : 16) + 4 * lw;  // this wave's 4 Q blocks
  const int pblk0 = (xside ? 16 : 0) + 4 * lw;  // and 4 P blocks (X: bottom half, Y: top half)
  // the walk of contract_tile
  const int row_end = min(m0 + C::BM, args.M);
  const int ecol = STK == 1 ? __builtin_amdgcn_readfirstlane((n0 / args.group_cols) * args.group_ecols) : 0;
  int grp = 0;
  int seg = -1;
  auto first_seg = [&]() {
    if (seg < 0) seg = args.E != nullptr ? seg_of_row(args.seg, m0) : args.seg.n;
  };
  KSource src{static_cast<const char *>(args.P), static_cast<const char *>(args.Q), 2 * args.ldp, 2 * args.ldq, 0,
              args.M, args.Kc, 2};
  constexpr int bk = C::KB / 2;
  int ntile = (src.klim + bk - 1) / bk;
  if (ntile == 0) {
    first_seg();
    if (!next_lora_source(args, C::NN, m0, row_end, seg, src, ecol)) return;
    ntile = (src.klim + bk - 1) / bk;
  }
  bool kmask = ntile * bk != src.klim;
  PPLoad<C> lq, lp;
  lq.init_q(src, n0, args.Ncols, lane);
  lp.init_p(src, m0, lane);
  bool lp_stale = false;  // X: lp is to follow the walk's source at the next step
  int t_in_src = 0, n_real = 1;
  bool exhausted = false;
  auto repoint = [&]() {
    lq.init_q(src, n0, args.Ncols, lane);
    if (xside) lp_stale = true;
    else lp.init_p(src, m0, lane);
  };
  auto advance = [&]() -> bool {
    if (exhausted) return false;
    if (t_in_src + 1 < ntile) {
      ++t_in_src;
      ++n_real;
      return true;
    }
    if constexpr (STK == 2) {
      if (grp + 1 < args.groups) {
        ++grp;
        src = KSource{reinterpret_cast<const char *>(args.Pg[grp]),
                      reinterpret_cast<const char *>(args.Q) + 2 * (int64_t)grp * args.group_cols, 2 * args.ldp,
                      2 * args.ldq, 0, args.M, args.group_cols, 2};
        kmask = src.klim % bk != 0;
        repoint();
        t_in_src = 0;
        ++n_real;
        return true;
      }
    }
    first_seg();
    if (!next_lora_source(args, C::NN, m0, row_end, seg, src, ecol)) {
      exhausted = true;
      return false;
    }
    ntile = (src.klim + bk - 1) / bk;
    kmask = src.klim % bk != 0;
    repoint();
    t_in_src = 0;
    ++n_real;
    return true;
  };
  // this wave's 4 blocks (from blk0) of a k-tile of loader l into the LDS tile at `base` (P: a
  // 128-row half slot, block blk at (blk & 15) KB). The destinations are this wave's block
  // offset, taken opaque where it is used, plus constants: one scalar add per load instead of
  // dozens of precomputed addresses that do not fit the scalar registers.
  auto issue4 = [&](auto is_p, const PPLoad<C> &l, MLORA_LDS char *base, int blk0, int k0, bool km, bool live) {
    constexpr bool ISP = decltype(is_p)::value;
    MLORA_LDS char *wb = base + opaque_sgpr(1024 * (ISP ? blk0 & 15 : blk0));
    if (l.masked(km, live)) {
#pragma unroll
      for (int q = 0; q < 4; ++q) l.template issue<true>(wb + 1024 * q, blk0 + q, k0, km, live, lane);
    } else {
#pragma unroll
      for (int q = 0; q < 4; ++q) l.template issue<false>(wb + 1024 * q, blk0 + q, k0, km, live, lane);
    }
  };
  auto issue_q = [&](MLORA_LDS char *base, int k0, bool km, bool live) {
    issue4(std::false_type{}, lq, base, qblk0, k0, km, live);
  };
  auto issue_p = [&](MLORA_LDS char *base, int k0, bool km, bool live) {
    issue4(std::true_type{}, lp, base, pblk0, k0, km, live);
  };
  // this lane's fragment offsets in substep h (P: within a half slot; see FragAddr)
  int32_t fa[NSUB], fb[NSUB];
  {
    const int z = swzk<C::CPR>(lane & 31);
#pragma unroll
    for (int h = 0; h < NSUB; ++h) {
      const int slot = (2 * h + (lane >> 5)) ^ z;
      fa[h] = ((wm0 & 127) + (lane & 31)) * C::KB + 16 * slot;
      fb[h] = (wn0 + (lane & 31)) * C::KB + 16 * slot;
    }
  }
  Half<C> f[NSUB];
  // fragment offset o moved by a multiple of 64 KB (the part of an LDS offset past the 16-bit
  // immediate of a ds_read): added in the phase that reads, not held across the loop, and kept
  // apart from the immediates that follow
  auto hi = [](int32_t o, int add) -> int32_t { return add == 0 ? o : opaque_vgpr(opaque_vgpr(o) + add); };
  // all of this wave's fragments of the k-tile in phase PH (P from the half slots at PBASE)
  auto read_tile = [&](auto ph_c, auto pbase_c) {
    constexpr int PH = decltype(ph_c)::value;
    constexpr int PO = decltype(pbase_c)::value + (PH % 2) * 16384, QO = QB + (PH % 3) * 32768;
    static_for<NSUB>([&](auto h_c) {
      constexpr int H = decltype(h_c)::value;
      const int32_t pa = hi(fa[H], PO & ~65535);
#pragma unroll
      for (int i = 0; i < C::TM; ++i) f[H].a[i] = *(const lds_u4 *)(lds + pa + (PO & 65535) + 32 * C::KB * i);
      const int32_t qa = hi(fb[H], QO & ~65535);
#pragma unroll
      for (int j = 0; j < C::TN; ++j) f[H].b[j] = *(const lds_u4 *)(lds + qa + (QO & 65535) + 32 * C::KB * j);
      return true;
    });
  };
  auto compute = [&]() {
#pragma unroll
    for (int h = 0; h < NSUB; ++h)
#pragma unroll
      for (int g = 0; g < C::TMN; ++g) {
        const int j = g / C::TM, i = g % C::TM;
        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(as_bf16x8(f[h].b[j]), as_bf16x8(f[h].a[i]), acc[i][j], 0, 0, 0);
      }
  };
  // k-tiles of the main contraction that need no mask (all but a partial last one): the steps
  // whose loads read only those run in a loop of their own, without the walk and the mask
  // decisions, so the phases that issue loads carry no more than the loads and reads themselves;
  // the walk takes over, at k-tile t + 1, in the phase where that loop stopped
  const int n_full = STK == 2 ? 0 : args.Kc / bk;
  int t = 0;
  bool done = false;
  // prologue: k-tiles 0 and 1 of this side's loads; the walk ends at k-tile 1
  issue_q(lds + QB, 0, kmask, true);
  issue_p(lds + (xside ? PB : PT), 0, kmask, true);
  const bool live1 = advance();
  issue_q(lds + QB + 32768, t_in_src * bk, kmask, live1);
  if (xside) {
    wait_vmcnt<8>();  // Q(0) blocks 0-15
    phase_barrier();
    bool live_prev = live1;  // whether k-tile t + 1 (the walk's) exists
    while (t + 2 < n_full) static_for<PER>([&](auto st) -> bool {  // Q(t+2) and Pbot(t+1) main
        constexpr int ST = decltype(st)::value;
        if (t + 2 >= n_full) return false;
        issue_q(lds + QB + ((ST + 2) % 3) * 32768, (t + 2) * bk, false, true);
        issue_p(lds + PB + ((ST + 1) % 2) * 16384, (t + 1) * bk, false, true);
        read_tile(st, std::integral_constant<int, PT>{});
        wait_vmcnt<8>();  // this wave's loads of the phase before
        phase_barrier();
        compute();
        phase_barrier();
        ++t;
        return true;
      });
    if (n_full >= 2) {  // the walk at k-tile t + 1 (the main contraction)
      t_in_src = t + 1;
      n_real = t + 2;
    }
    const int st0 = t % PER;
    bool first = true;
    while (!done) static_for<PER>([&](auto st) -> bool {
        constexpr int ST = decltype(st)::value;
        if (first && ST < st0) return true;  // the walk starts where the main loop stopped
        first = false;
        if (lp_stale) {  // the P loads of this step read k-tile t + 1, the walk's
          lp.init_p(src, m0, lane);
          lp_stale = false;
        }
        const int k0_p = t_in_src * bk;
        const bool km_p = kmask, live_p = live_prev;
        const bool live = advance();  // k-tile t + 2
        issue_q(lds + QB + ((ST + 2) % 3) * 32768, t_in_src * bk, kmask, live);
        issue_p(lds + PB + ((ST + 1) % 2) * 16384, k0_p, km_p, live_p);
        live_prev = live;
        read_tile(st, std::integral_constant<int, PT>{});
        wait_vmcnt<8>();
        phase_barrier();
        compute();
        if (t + 1 >= n_real) wait_vmcnt<0>();  // last k-tile: every load drained before the last barrier
        phase_barrier();
        ++t;
        done = t >= n_real;
        return !done;
      });
    // no barrier for Y's last MFMA phase: every wave's reads and loads are done, and the
    // epilogue stages rows 0-127 (X) and 128-255 (Y) without a workgroup barrier
  } else {
    issue_p(lds + PT + 16384, t_in_src * bk, kmask, live1);
    wait_vmcnt<8>();  // Q(0) blocks 16-31, Ptop(0)
    phase_barrier();
    phase_barrier();  // X reads k-tile 0
    while (t + 2 < n_full) static_for<PER>([&](auto st) -> bool {  // Q(t+2) and Ptop(t+2) main
        constexpr int ST = decltype(st)::value;
        if (t + 2 >= n_full) return false;
        issue_q(lds + QB + ((ST + 2) % 3) * 32768, (t + 2) * bk, false, true);
        issue_p(lds + PT + (ST % 2) * 16384, (t + 2) * bk, false, true);
        read_tile(st, std::integral_constant<int, PB>{});
        wait_vmcnt<8>();
        phase_barrier();
        compute();
        phase_barrier();
        ++t;
        return true;
      });
    if (n_full >= 2) {
      t_in_src = t + 1;
      n_real = t + 2;
    }
    const int st0 = t % PER;
    bool first = true;
    while (!done) static_for<PER>([&](auto st) -> bool {
        constexpr int ST = decltype(st)::value;
        if (first && ST < st0) return true;
        first = false;
        const bool live = advance();  // k-tile t + 2
        issue_q(lds + QB + ((ST + 2) % 3) * 32768, t_in_src * bk, kmask, live);
        issue_p(lds + PT + (ST % 2) * 16384, t_in_src * bk, kmask, live);
        read_tile(st, std::integral_constant<int, PB>{});
        const bool last = t + 1 >= n_real;
        if (last) wait_vmcnt<0>();  // every load drained before the last barrier
        else wait_vmcnt<8>();
        phase_barrier();
        compute();
        if (!last) phase_barrier();
        ++t;
        done = t >= n_real;
        return !done;
      });
  }
  wait_vmcnt<0>();
}

// Output tile of physical index p: XCD-contiguous logical ids (workgroups
// are dealt round-robin over the 8 XCDs), then groups of group_m row-tiles
// walked column by column so concurrently running tiles share P rows and Q
// columns in L2.
template <int BM, int BN>
__device__ __forceinline__ void tile_origin(const GemmArgs &args, int p, int &m0, int &n0) {
  const int nblocks = args.tiles_m * args.tiles_n;
  const int id = xcd_remap(p, nblocks);
  const int per_group = args.group_m * args.tiles_n;
  const int group = id / per_group;
  const int first_m = group * args.group_m;
  const int gsize = min(args.tiles_m - first_m, args.group_m);
  const int tm = first_m + (id % per_group) % gsize;
  const int tn = (id % per_group) / gsize;
  m0 = tm * BM;
  n0 = tn * BN;
}

// This lane's 4 entries of a per-column vector (bf16 when BF16, else f32) at columns c .. c + 3
// (c a multiple of 4): one 8- or 16-byte load; past the vector's end (Ncols is a multiple of 8,
// so a group of 4 is all in range or all past it) the buffer reads zeros.
template <bool BF16>
__device__ __forceinline__ f32x4 cols4(__amdgpu_buffer_rsrc_t r, int c) {
  if constexpr (BF16) {
    const uint2 w = __builtin_bit_cast(uint2, __builtin_amdgcn_raw_buffer_load_b64(r, 2 * c, 0, 0));
    return f32x4{bf16_to_f32(w.x & 0xffff), bf16_to_f32(w.x >> 16), bf16_to_f32(w.y & 0xffff), bf16_to_f32(w.y >> 16)};
  } else {
    return __builtin_bit_cast(f32x4, buf_load16(r, 4 * c));
  }
}

// x + y·g of the reference's gated residual: fp32 multiply, then fp32 add, each
// rounded to nearest (no fused multiply-add), as runtime/helios_residual_kernel.py:66-86
// states it.
__device__ __forceinline__ float gated_add(float x, float y, float g) {
#pragma clang fp contract(off)
  const float p = y * g;
  return x + p;
}

// Epilogue of one output tile: (fp8: x_scale[m]·w_scale[n]), + bias, (+ Y), round to bf16.
// Register 4g + e of tile (i, j) holds row m = m0 + wm0 + 32i + lane%32 and column
// n = n0 + wn0 + 32j + 8g + 4(lane/32) + e. BK: the bias (0: none, 1: bf16, 2: f32).
// The bias and column scales come in as this lane's own 4-column groups (vector loads).
template <class C>
struct EpiVectors {
  __amdgpu_buffer_rsrc_t rb, rq;
  bool has_qs;
  float ps[C::TM];  // fp8: x_scale of each row tile's row
  __device__ __forceinline__ void init(const GemmArgs &args, int bk, int m0, int wm0, int lane) {
    rb = make_rsrc(args.bias, bk ? (int64_t)args.Ncols * (bk == 1 ? 2 : 4) : 0);
    has_qs = C::F8 && args.qsc != nullptr;
    rq = make_rsrc(args.qsc, has_qs ? (int64_t)args.Ncols * 4 : 0);
#pragma unroll
    for (int i = 0; i < C::TM; ++i) {
      const int m = m0 + wm0 + 32 * i + (lane & 31);
      ps[i] = 1.f;
      if constexpr (C::F8) ps[i] = m < args.M ? args.psc[m] : 0.f;
    }
  }
  // the 4 values of tile (i, j), group g, scaled (fp8) and biased, as fp32
  template <int BK>
  __device__ __forceinline__ void apply(float (&v)[4], const f32x16 &a, int g, int i, const f32x4 &b4,
                                        const f32x4 &q4) const {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      v[e] = a[4 * g + e];
      // e4m3: acc = Σ xq·wq + Σ (h/x_scale)·(B/w_scale): one scaling restores both
      if constexpr (C::F8) v[e] *= ps[i] * q4[e];
      if constexpr (BK != 0) v[e] += b4[e];
    }
  }
  template <int BK>
  __device__ __forceinline__ void load(f32x4 &b4, f32x4 &q4, int c) const {
    b4 = f32x4{0.f, 0.f, 0.f, 0.f};
    if constexpr (BK != 0) b4 = cols4<BK == 1>(rb, c);
    q4 = f32x4{1.f, 1.f, 1.f, 1.f};
    if constexpr (C::F8) {
      if (has_qs) q4 = cols4<false>(rq, c);
    }
  }
};

// Staged store: the rounded tile goes to LDS (whose operand stages must be free), row-major with
// 16-byte chunk q of row r at slot q ^ (r % CH), and leaves in 16-byte stores that cover whole
// rows. Lane l writes its 8 bytes of (i, j, g) to row wm0 + 32i + l%32, slot
// (wn0/8 + 4j + g) ^ (l%32 % CH): one XOR per (j, g), the row part an immediate offset.
template <class C, int BK, bool RESID>
__device__ __forceinline__ void store_staged(const f32x16 (&acc)[C::TM][C::TN], const GemmArgs &args,
                                             MLORA_LDS char *lds, int m0, int n0, int wm0, int wn0, int lane,
                                             uint16_t *Ybase, int ncol0) {
  constexpr int ROWB = C::BN * 2;  // bytes per staged row
  constexpr int CH = C::BN / 8;    // 16-byte chunks per staged row
  static_assert(C::LDS_BYTES >= C::BM * ROWB, "the staged output tile fits the operand stages");
  static_assert(C::WM * 32 * C::TM == C::BM && (C::BM / C::WM) % 32 == 0, "row tiles of 32 rows");
  const int l31 = lane & 31, hh = lane >> 5;
  const int ncol = n0 + wn0 + 4 * hh;  // this lane's first column of tile 0, group 0
  EpiVectors<C> ev;
  ev.init(args, BK, m0, wm0, lane);
  // bf16 bias: every entry this lane needs (TN x 4 groups), loaded before the barrier
  f32x4 b0[BK == 1 ? C::TN * 4 : 1];
  if constexpr (BK == 1) {
#pragma unroll
    for (int q = 0; q < C::TN * 4; ++q) b0[q] = cols4<true>(ev.rb, ncol + 8 * q);
  }
  // every wave's operand loads have landed and been read (the ping-pong schedule ensures that
  // for the rows a wave stages by the time it leaves its k-loop)
  if constexpr (!C::PP) lds_pipeline_barrier();
  else asm volatile("" ::: "memory");
  const int rowb = (wm0 + l31) * ROWB + 8 * hh;
  const int w8 = wn0 >> 3;
  const int z = l31 % CH;
#pragma unroll
  for (int j = 0; j < C::TN; ++j) {
    f32x4 b4[4], q4[4];
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      ev.template load<BK == 1 ? 0 : BK>(b4[g], q4[g], ncol + 32 * j + 8 * g);
      if constexpr (BK == 1) b4[g] = b0[4 * j + g];
    }
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      MLORA_LDS char *dst = lds + rowb + 16 * ((w8 + 4 * j + g) ^ z);
#pragma unroll
      for (int i = 0; i < C::TM; ++i) {
        float v[4];
        ev.template apply<BK>(v, acc[i][j], g, i, b4[g], q4[g]);
        *(MLORA_LDS u32x2 *)(dst + i * 32 * ROWB) = u32x2{pack2_bf16(v[0], v[1]), pack2_bf16(v[2], v[3])};
      }
    }
  }
  // Each wave stores the block it staged itself: (BM / WM) rows of (BN / WN) columns, in 1 KB
  // instructions of whole 16-byte chunks. It reads only its own LDS writes, so a wave-level
  // ordering suffices (no workgroup barrier).
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  const int rows_here = min(C::BM, args.M - m0);
  const int64_t ldy_b = args.ldy * 2;
  const __amdgpu_buffer_rsrc_t ry = make_rsrc(Ybase + (int64_t)m0 * args.ldy, rows_here * ldy_b);
  constexpr int WROWS = C::BM / C::WM, WCH = C::BN / C::WN / 8;  // the wave's rows; its 16-byte chunks per row
  constexpr int RPI = 64 / WCH;                                  // rows per 1 KB instruction
  static_assert(64 % WCH == 0 && WROWS % RPI == 0, "whole store instructions per wave");
#pragma unroll
  for (int it = 0; it < WROWS / RPI; ++it) {
    const int r = wm0 + it * RPI + lane / WCH;
    const int q = w8 + lane % WCH;
    u32x4 d = *(const lds_u4 *)(lds + r * ROWB + 16 * (q ^ (r % CH)));
    const int n = n0 + 8 * q;
    const int32_t off = (r < rows_here && n < args.Ncols) ? (int32_t)(r * ldy_b + (n - ncol0) * 2) : kOOB;
    if constexpr (RESID) {
      // the 8 bf16 values of d are bf16(Y); x and gate of the same 8 columns
      if (off != kOOB) {
        const int64_t m = m0 + r;
        const MLORA_GLOBAL f32x4 *gp = (const MLORA_GLOBAL f32x4 *)(args.gate + (m / args.gate_rows) * args.ldgate + n);
        const f32x4 g0 = gp[0], g1 = gp[1];
        float xs[8];
        if (args.res_f32) {
          const MLORA_GLOBAL f32x4 *xp = (const MLORA_GLOBAL f32x4 *)((const float *)args.res + m * args.ldres + n);
          const f32x4 x0 = xp[0], x1 = xp[1];
#pragma unroll
          for (int e = 0; e < 4; ++e) xs[e] = x0[e], xs[e + 4] = x1[e];
        } else {
          const u32x4 xv = *(const MLORA_GLOBAL u32x4 *)((const uint16_t *)args.res + m * args.ldres + n);
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            const uint32_t xw = xv[e / 2];
            xs[e] = bf16_to_f32((uint16_t)(e % 2 ? xw >> 16 : xw & 0xffff));
          }
        }
        float o[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const uint32_t yw = d[e / 2];
          const float y = bf16_to_f32((uint16_t)(e % 2 ? yw >> 16 : yw & 0xffff));
          o[e] = gated_add(xs[e], y, e < 4 ? g0[e] : g1[e - 4]);
        }
        if (args.res_f32) {
          // float32 stream: no bf16 rounding of the sum; 32 bytes per lane
          MLORA_GLOBAL f32x4 *op = (MLORA_GLOBAL f32x4 *)(args.Yf + m * args.ldy + n);
          op[0] = f32x4{o[0], o[1], o[2], o[3]};
          op[1] = f32x4{o[4], o[5], o[6], o[7]};
          continue;
        }
#pragma unroll
        for (int e = 0; e < 4; ++e) d[e] = pack2_bf16(o[2 * e], o[2 * e + 1]);
      } else if (args.res_f32) {
        continue;
      }
    }
    buf_store16_nt(ry, off, d);
  }
}

// Direct store (accumulating into Y, which adds the old value in fp32 before the one rounding):
// each lane stores its 4 consecutive columns of (i, j, g).
template <class C, int BK>
__device__ __forceinline__ void store_direct(const f32x16 (&acc)[C::TM][C::TN], const GemmArgs &args, int m0, int n0,
                                             int wm0, int wn0, int lane, uint16_t *Ybase, int ncol0) {
  const int rows_here = min(C::BM, args.M - m0);
  const int64_t ldy_b = args.ldy * 2;
  const __amdgpu_buffer_rsrc_t ry = make_rsrc(Ybase + (int64_t)m0 * args.ldy, rows_here * ldy_b);
  const int ncol = n0 + wn0 + 4 * (lane >> 5);
  EpiVectors<C> ev;
  ev.init(args, BK, m0, wm0, lane);
#pragma unroll
  for (int j = 0; j < C::TN; ++j) {
    f32x4 b4[4], q4[4];
#pragma unroll
    for (int g = 0; g < 4; ++g) ev.template load<BK>(b4[g], q4[g], ncol + 32 * j + 8 * g);
#pragma unroll
    for (int i = 0; i < C::TM; ++i) {
      const int ml = wm0 + 32 * i + (lane & 31);
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int n = ncol + 32 * j + 8 * g;
        float v[4];
        ev.template apply<BK>(v, acc[i][j], g, i, b4[g], q4[g]);
        // rows past M / columns past Ncols fall outside ry or are dropped
        const int32_t off = (ml < rows_here && n < args.Ncols) ? (int32_t)(ml * ldy_b + (n - ncol0) * 2) : kOOB;
        if (args.accumulate && off != kOOB) {
          const u32x2 o = *(const MLORA_GLOBAL u32x2 *)(Ybase + (int64_t)(m0 + ml) * args.ldy + (n - ncol0));
          v[0] += bf16_to_f32(o.x & 0xffff); v[1] += bf16_to_f32(o.x >> 16);
          v[2] += bf16_to_f32(o.y & 0xffff); v[3] += bf16_to_f32(o.y >> 16);
        }
        buf_store8(ry, off, make_uint2(pack2_bf16(v[0], v[1]), pack2_bf16(v[2], v[3])));
      }
      __builtin_amdgcn_sched_barrier(0);  // one accumulator tile at a time
    }
  }
}

// Ybase: the output matrix (pitch ldy); its column 0 is tile column ncol0 (a stacked linear's
// first column; 0 otherwise). RESID: the stored value is the block's gated residual of bf16(Y)
// (staged path only: the gated-residual entry points never accumulate).
template <class C, bool RESID>
__device__ __forceinline__ void store_tile(const f32x16 (&acc)[C::TM][C::TN], const GemmArgs &args, MLORA_LDS char *lds,
                                           int m0, int n0, int wm0, int wn0, int lane, uint16_t *Ybase, int ncol0) {
  if (!RESID && args.accumulate) {
    if (args.bias_dtype == MLORA_BF16) store_direct<C, 1>(acc, args, m0, n0, wm0, wn0, lane, Ybase, ncol0);
    else if (args.bias_dtype == MLORA_F32) store_direct<C, 2>(acc, args, m0, n0, wm0, wn0, lane, Ybase, ncol0);
    else store_direct<C, 0>(acc, args, m0, n0, wm0, wn0, lane, Ybase, ncol0);
    return;
  }
  if (args.bias_dtype == MLORA_BF16) store_staged<C, 1, RESID>(acc, args, lds, m0, n0, wm0, wn0, lane, Ybase, ncol0);
  else if (args.bias_dtype == MLORA_F32) store_staged<C, 2, RESID>(acc, args, lds, m0, n0, wm0, wn0, lane, Ybase, ncol0);
  else store_staged<C, 0, RESID>(acc, args, lds, m0, n0, wm0, wn0, lane, Ybase, ncol0);
}

// One workgroup per output tile. RESID: the stored value is the block's gated
// residual of the result (see store_tile). STK: stacked linears (see GemmArgs).
template <class C, bool RESID = false, int STK = 0>
__global__ __launch_bounds__(C::THREADS, C::WAVES_PER_SIMD) void gemm_kernel(const GemmArgs args) {
  __shared__ u32x4 smem[C::LDS_BYTES / 16];
  MLORA_LDS char *lds = (MLORA_LDS char *)smem;
  const int tid = threadIdx.x, lane = tid & 63, wave = wave_id();
  // the scalar arguments of the tile order and the first k-tile loads, fetched together (one
  // wait) instead of one dependent fetch after another
  asm volatile("" ::"s"(args.tiles_m), "s"(args.tiles_n), "s"(args.group_m), "s"(args.M), "s"(args.Ncols),
               "s"(args.Kc), "s"(args.ldp), "s"(args.ldq), "s"(args.P), "s"(args.Q));
  const int wm0 = (wave / C::WN) * (C::BM / C::WM);
  const int wn0 = (wave % C::WN) * (C::BN / C::WN);
  int m0, n0;
  if (C::BM == 128 && C::BN == 128 && args.tail_base >= 0) {
    // quarter q of the 256x256 tile tail_base + blockIdx.x / 4; a quarter wholly past the
    // matrix (a narrow last row or column tile) has nothing to compute or store
    const int q = blockIdx.x % 4;
    tile_origin<256, 256>(args, args.tail_base + (int)blockIdx.x / 4, m0, n0);
    m0 += 128 * (q / 2);
    n0 += 128 * (q % 2);
    if (m0 >= args.M || n0 >= args.Ncols) return;  // uniform over the workgroup, before any barrier
  } else {
    tile_origin<C::BM, C::BN>(args, blockIdx.x, m0, n0);
  }
  f32x16 acc[C::TM][C::TN];
#pragma unroll
  for (int i = 0; i < C::TM; ++i)
#pragma unroll
    for (int j = 0; j < C::TN; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.f;
  if constexpr (C::PP) {
    contract_tile_pp<C, STK>(acc, args, lds, wm0, wn0, m0, n0, tid);
  } else {
    FragAddr<C> fa;
    fa.init(wm0, wn0, lane);
    contract_tile<C, STK>(acc, args, lds, fa, m0, n0, tid);
  }
  if constexpr (STK == 1) {
    const int g = __builtin_amdgcn_readfirstlane(n0 / args.group_cols);
    store_tile<C, RESID>(acc, args, lds, m0, n0, wm0, wn0, lane, args.Yg[g], g * args.group_cols);
  } else {
    store_tile<C, RESID>(acc, args, lds, m0, n0, wm0, wn0, lane, args.Y, 0);
  }
}

using CfgNT256 = GemmCfg<256, 256, 4, 2, false, false, 128, 2, true, true, true>;
using CfgF8256 = GemmCfg<256, 256, 4, 2, false, true, 128, 2, true, true>;
using CfgF8128 = GemmCfg<128, 128, 2, 2, false, true>;
using CfgNN256 = GemmCfg<256, 256, 4, 2, true, false, 128, 2, true, true>;
using CfgNT128 = GemmCfg<128, 128, 2, 2, false>;
using CfgNN128 = GemmCfg<128, 128, 2, 2, true>;
// 128x128 tiles of 8 waves (32x64 each) with three stages (two k-tiles in flight), one workgroup
// per CU: grids of at most 256 such tiles, and the quarters of a partly filled last round of
// 256x256 tiles (dispatch_gemm)
using CfgNT128W = GemmCfg<128, 128, 4, 2, false, false, 128, 3>;
using CfgNN128W = GemmCfg<128, 128, 4, 2, true, false, 128, 3>;

// Row tiles per group of the tile order: an XCD's 32 concurrent 256x256 tiles
// then cover 4 row tiles x up to 8 column tiles (P, streamed from HBM, shared
// by more tiles; Q, smaller and mostly held in the last-level cache, by fewer).
// Measured against groups of 8 and 2: 1-1.5% faster than 8 on all three Wan
// shapes, bit-equal output.
constexpr int kGroupM = 4;

// One workgroup per tile of C's size, the first `nblocks` of the tile order (all when < 0).
template <class C, bool RESID = false, int STK = 0>
static int launch_gemm(GemmArgs &a, hipStream_t stream, int64_t nblocks = -1) {
  a.tiles_m = (a.M + C::BM - 1) / C::BM;
  a.tiles_n = (a.Ncols + C::BN - 1) / C::BN;
  a.tail_base = -1;
  if (a.group_m <= 0) a.group_m = kGroupM;
  if (nblocks < 0) nblocks = (int64_t)a.tiles_m * a.tiles_n;
  if (nblocks == 0) return MLORA_OK;
  if (nblocks > INT32_MAX) return MLORA_ERR_LIMIT;
  hipLaunchKernelGGL((gemm_kernel<C, RESID, STK>), dim3((unsigned)nblocks), dim3(C::THREADS), 0, stream, a);
  return launch_status();
}

// The 256x256 tiles from `first` on, as 128x128 quarters of configuration Q.
template <class Q, bool RESID = false, int STK = 0>
static int launch_tail(GemmArgs &a, hipStream_t stream, int64_t first) {
  static_assert(Q::BM == 128 && Q::BN == 128, "quarters of 256x256 tiles");
  a.tiles_m = (a.M + 255) / 256;
  a.tiles_n = (a.Ncols + 255) / 256;
  const int64_t tail = (int64_t)a.tiles_m * a.tiles_n - first;
  a.tail_base = (int32_t)first;
  if (a.group_m <= 0) a.group_m = kGroupM;
  hipLaunchKernelGGL((gemm_kernel<Q, RESID, STK>), dim3((unsigned)(4 * tail)), dim3(Q::THREADS), 0, stream, a);
  return launch_status();
}

// Tile choice (measured on MI355X):
// * At least 256 tiles of 256x256: the 8-wave 256x256 tile (the persistent form whose k-tile ring
//   runs across output tiles, and 256x128 tiles with a 3-stage ring, both measured slower).
// * Fewer, and at most 256 tiles of 128x128: one 8-wave 128x128 workgroup per CU with three
//   stages (CfgNT128W / CfgNN128W), 15-35% faster than the 4-wave two-stage tile, two per CU, at
//   48-192 tiles (512-2048 rows, K 1536-8960); with more tiles (two rounds or more of one
//   workgroup per CU) it measured 2-32% slower (7% faster only for a forward at K = 3072).
// * Otherwise the 4-wave two-stage 128x128 tile, two workgroups per CU.
// A grid of 256x256 tiles a little over whole rounds of the 256 CUs (1284 tiles at 27280 x 3072:
// five rounds and four tiles) would spend a whole tile's time on its last few tiles. Those
// tiles (at most 64, the last of the tile order) then run in a second launch as 128x128
// quarters of the 8-wave configuration, one round of at most 256 workgroups: config 3's
// 27280 x 3072 forward and NN dX took 10% and 7% less time per launch, its step 2.9% less.
// (The 4-wave two-stage 128x128 tile was no faster than no split. Tails of 104 and 128 tiles,
// two rounds of quarters, were 2-6% faster per launch in isolation but left config 4's step
// 0.6% slower.) Every output keeps the same k order and MFMA sequence in all tile sizes, so
// the result is the same bit for bit. The e4m3 GEMM keeps the 4-wave 128x128 tile for small
// grids and its tail as 256x256 tiles (its 8-wave quarters measured 1% slower).
template <class Big, class Small, bool RESID = false, int STK = 0>
static int dispatch_gemm(GemmArgs &a, hipStream_t stream) {
  constexpr int64_t kCUs = 256, kMaxTail = 64;
  using Wide = std::conditional_t<Big::F8, void, std::conditional_t<Big::NN, CfgNN128W, CfgNT128W>>;
  const int64_t big_tiles = (int64_t)((a.M + 255) / 256) * ((a.Ncols + 255) / 256);
  if (big_tiles < kCUs) {
    if constexpr (!std::is_void_v<Wide>) {
      const int64_t tiles = (int64_t)((a.M + 127) / 128) * ((a.Ncols + 127) / 128);
      if (tiles <= kCUs) return launch_gemm<Wide, RESID, STK>(a, stream);
    }
    return launch_gemm<Small, RESID, STK>(a, stream);
  }
  const int64_t tail = big_tiles % kCUs;
  if constexpr (std::is_void_v<Wide>) {
    return launch_gemm<Big, RESID, STK>(a, stream);
  } else {
    if (tail == 0 || tail > kMaxTail) return launch_gemm<Big, RESID, STK>(a, stream);
    const int st = launch_gemm<Big, RESID, STK>(a, stream, big_tiles - tail);
    if (st) return st;
    return launch_tail<Wide, RESID, STK>(a, stream, big_tiles - tail);
  }
}

static int fill_common(GemmArgs &a, int64_t M, int64_t Kc, int64_t Ncols, const void *e, int64_t lde,
                       const void *const *ext_ptrs, const int32_t *ranks, int32_t n_adapters, const int64_t *seg_offsets,
                       const int32_t *adapter_ids, int32_t n_segments) {
  if (M < 0 || Kc < 0 || Ncols < 0) return MLORA_ERR_INVALID;
  if (M > INT32_MAX - 1024 || Kc > INT32_MAX - 1024 || Ncols > INT32_MAX - 1024) return MLORA_ERR_LIMIT;
  int st = build_segtable(a.seg, M, seg_offsets, adapter_ids, n_segments, n_adapters);
  if (st) return st;
  st = build_adapters(a.ext, a.seg, ext_ptrs, ranks, nullptr, n_adapters, kMaxGemmRank);
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

extern "C" int mlora_gemm_fwd_stacked(const void *x, int64_t ldx, int64_t M, int64_t K, const void *w, int64_t ldw,
                                      int64_t N, int64_t group_cols, const void *bias, int bias_dtype,
                                      const void *h_rows, int64_t ldh, int64_t group_ecols,
                                      const void *const *b_ptrs, const int32_t *ranks, int32_t n_adapters,
                                      const int64_t *seg_offsets, const int32_t *adapter_ids, int32_t n_segments,
                                      void *const *y_ptrs, int64_t ldy, void *stream) {
  GemmArgs a{};
  int st = fill_common(a, M, K, N, h_rows, ldh, b_ptrs, ranks, n_adapters, seg_offsets, adapter_ids, n_segments);
  if (st) return st;
  if (group_cols <= 0 || group_cols % 256 != 0 || N % group_cols != 0 || N / group_cols > MLORA_MAX_STACKED)
    return MLORA_ERR_UNSUPPORTED;
  const int64_t groups = N / group_cols;
  if ((st = check_bf16_matrix(x, ldx, M, K))) return st;
  if ((st = check_bf16_matrix(w, ldw, N, K))) return st;
  if (y_ptrs == nullptr) return MLORA_ERR_INVALID;
  for (int64_t g = 0; g < groups; ++g)
    if ((st = check_bf16_matrix(y_ptrs[g], ldy, M, group_cols))) return st;
  const int rmax = max_used_rank(a.seg, a.ext);
  if (group_ecols < 0 || group_ecols % 8 != 0 || rmax > group_ecols) return MLORA_ERR_INVALID;
  if (rmax > 0 && (ldh < groups * group_ecols)) return MLORA_ERR_INVALID;  // every linear's LoRA columns
  if (M == 0 || N == 0) return MLORA_OK;
  for (int64_t g = 0; g < groups; ++g)
    if (y_ptrs[g] == nullptr) return MLORA_ERR_INVALID;
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
  a.Y = static_cast<uint16_t *>(y_ptrs[0]);
  a.ldy = ldy;
  a.groups = (int32_t)groups;
  a.group_cols = (int32_t)group_cols;
  a.group_ecols = (int32_t)group_ecols;
  for (int64_t g = 0; g < groups; ++g) a.Yg[g] = static_cast<uint16_t *>(y_ptrs[g]);
  return dispatch_gemm<CfgNT256, CfgNT128, false, 1>(a, static_cast<hipStream_t>(stream));
}

extern "C" int mlora_gemm_dx_stacked(const void *const *dy_ptrs, int64_t lddy, int64_t M, int64_t group_cols,
                                     int64_t groups, const void *w_t, int64_t ldw, int64_t K, const void *g_rows,
                                     int64_t ldg, const void *const *a_ptrs, const int32_t *ranks, int32_t n_adapters,
                                     const int64_t *seg_offsets, const int32_t *adapter_ids, int32_t n_segments,
                                     void *dx, int64_t lddx, void *stream) {
  GemmArgs a{};
  if (groups < 1 || groups > MLORA_MAX_STACKED || group_cols < 0) return MLORA_ERR_UNSUPPORTED;
  // contraction group_cols per linear (the main source of the kernel is linear 0's), output columns K
  int st = fill_common(a, M, group_cols, K, g_rows, ldg, a_ptrs, ranks, n_adapters, seg_offsets, adapter_ids,
                       n_segments);
  if (st) return st;
  if (dy_ptrs == nullptr) return MLORA_ERR_INVALID;
  for (int64_t g = 0; g < groups; ++g)
    if ((st = check_bf16_matrix(dy_ptrs[g], lddy, M, group_cols))) return st;
  if ((st = check_bf16_matrix(w_t, ldw, K, groups * group_cols))) return st;
  if ((st = check_bf16_matrix(dx, lddx, M, K))) return st;
  if (M == 0 || K == 0) return MLORA_OK;
  if (dx == nullptr) return MLORA_ERR_INVALID;
  for (int64_t g = 0; g < groups; ++g)
    if (group_cols > 0 && dy_ptrs[g] == nullptr) return MLORA_ERR_INVALID;
  if (!offsets_fit(lddy, 256) || !offsets_fit(lddx, 256) || !offsets_fit(ldw, 256)) return MLORA_ERR_LIMIT;
  a.P = static_cast<const uint16_t *>(dy_ptrs[0]);
  a.Q = static_cast<const uint16_t *>(w_t);
  a.ldp = lddy;
  a.ldq = ldw;
  a.bias = nullptr;
  a.bias_dtype = -1;
  a.Y = static_cast<uint16_t *>(dx);
  a.ldy = lddx;
  a.groups = (int32_t)groups;
  a.group_cols = (int32_t)group_cols;
  for (int64_t g = 0; g < groups; ++g) a.Pg[g] = static_cast<const uint16_t *>(dy_ptrs[g]);
  return dispatch_gemm<CfgNT256, CfgNT128, false, 2>(a, static_cast<hipStream_t>(stream));
}

extern "C" int mlora_gemm_fwd_gated(const void *x, int64_t ldx, int64_t M, int64_t K, const void *w, int64_t ldw,
                                    int64_t N, const void *bias, int bias_dtype, const void *h_rows, int64_t ldh,
                                    const void *const *b_ptrs, const int32_t *ranks, int32_t n_adapters,
                                    const int64_t *seg_offsets, const int32_t *adapter_ids, int32_t n_segments,
                                    const void *res, int64_t ldres, const float *gate, int64_t ldgate,
                                    int64_t gate_rows, void *out, int64_t ldout, int stream_dtype, void *stream) {
  GemmArgs a{};
  int st = fill_common(a, M, K, N, h_rows, ldh, b_ptrs, ranks, n_adapters, seg_offsets, adapter_ids, n_segments);
  if (st) return st;
  if (stream_dtype != MLORA_BF16 && stream_dtype != MLORA_F32) return MLORA_ERR_UNSUPPORTED;
  const bool f32 = stream_dtype == MLORA_F32;
  if ((st = check_bf16_matrix(x, ldx, M, K))) return st;
  if ((st = check_bf16_matrix(w, ldw, N, K))) return st;
  // the residual stream (res, out): bf16, or float32 rows of 16-byte chunks
  auto check_stream = [&](const void *p, int64_t ld) {
    if (!f32) return check_bf16_matrix(p, ld, M, N);
    if (M == 0 || N == 0) return (int)MLORA_OK;
    if (p == nullptr || ld < N) return (int)MLORA_ERR_INVALID;
    if (!aligned16(p) || ld % 4 != 0 || N % 8 != 0) return (int)MLORA_ERR_UNSUPPORTED;
    return (int)MLORA_OK;
  };
  if ((st = check_stream(res, ldres))) return st;
  if ((st = check_stream(out, ldout))) return st;
  if (M == 0 || N == 0) return MLORA_OK;
  if (out == nullptr || res == nullptr || gate == nullptr || gate_rows < 1 || gate_rows > INT32_MAX)
    return MLORA_ERR_INVALID;
  if (ldgate < N || ldgate % 4 != 0 || !aligned16(gate)) return MLORA_ERR_UNSUPPORTED;  // 16-byte gate rows
  if (bias != nullptr) {
    if (bias_dtype != MLORA_F32 && bias_dtype != MLORA_BF16) return MLORA_ERR_UNSUPPORTED;
    if (!aligned16(bias)) return MLORA_ERR_UNSUPPORTED;
  }
  // byte offsets of one tile's rows stay 31-bit (fp32 rows are twice as wide)
  if (!offsets_fit(ldx, 256) || !offsets_fit(ldout * (f32 ? 2 : 1), 256) || !offsets_fit(ldw, 256))
    return MLORA_ERR_LIMIT;
  a.P = static_cast<const uint16_t *>(x);
  a.Q = static_cast<const uint16_t *>(w);
  a.ldp = ldx;
  a.ldq = ldw;
  a.bias = bias;
  a.bias_dtype = bias ? bias_dtype : -1;
  // bf16 stream: Y is the output; float32 stream: the bf16 Y resource covers the same rows
  // (its offsets only gate which lanes store) and the values go to Yf
  a.Y = static_cast<uint16_t *>(out);
  a.ldy = ldout;
  a.Yf = f32 ? static_cast<float *>(out) : nullptr;
  a.res = res;
  a.ldres = ldres;
  a.gate = gate;
  a.ldgate = ldgate;
  a.gate_rows = (int32_t)gate_rows;
  a.res_f32 = f32 ? 1 : 0;
  return dispatch_gemm<CfgNT256, CfgNT128, true>(a, static_cast<hipStream_t>(stream));
}

extern "C" int mlora_gemm_dx(const void *dy, int64_t lddy, int64_t M, int64_t N, const void *w, int64_t ldw, int64_t K,
                             const void *g_rows, int64_t ldg, const void *const *a_ptrs, const int32_t *ranks,
                             int32_t n_adapters, const int64_t *seg_offsets, const int32_t *adapter_ids,
                             int32_t n_segments, void *dx, int64_t lddx, int accumulate, void *stream) {
  GemmArgs a{};
  // contraction over N, output columns K
  int st = fill_common(a, M, N, K, g_rows, ldg, a_ptrs, ranks, n_adapters, seg_offsets, adapter_ids, n_segments);
  if (st) return st;
  if ((st = check_bf16_matrix(dy, lddy, M, N))) return st;
  if ((st = check_bf16_matrix(w, ldw, N, K))) return st;
  if ((st = check_bf16_matrix(dx, lddx, M, K))) return st;
  if (M == 0 || K == 0) return MLORA_OK;
  if (dx == nullptr) return MLORA_ERR_INVALID;
  if (!offsets_fit(lddy, 256) || !offsets_fit(lddx, 256) || !offsets_fit(ldw, N) || !offsets_fit(K, kMaxGemmRank))
    return MLORA_ERR_LIMIT;
  a.P = static_cast<const uint16_t *>(dy);
  a.Q = static_cast<const uint16_t *>(w);
  a.ldp = lddy;
  a.ldq = ldw;
  a.bias = nullptr;
  a.bias_dtype = -1;
  a.Y = static_cast<uint16_t *>(dx);
  a.ldy = lddx;
  a.accumulate = accumulate ? 1 : 0;
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
  if (y == nullptr || xq == nullptr || wq == nullptr || x_scale == nullptr) return MLORA_ERR_INVALID;
  if (K == 0) return MLORA_ERR_UNSUPPORTED;  // the contraction loop starts with an e4m3 k-tile
  if (w_scale != nullptr && !aligned16(w_scale)) return MLORA_ERR_UNSUPPORTED;  // NULL: all 1
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
