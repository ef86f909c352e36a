// Segment-gathered LoRA kernels (HBM-bound): shrink and the adapter-gradient
// reductions.
//
// shrink     h[m, j]   = s_a · Σ_k P[m,k]·Op_a(j,k)           (X·Aᵀ forward, s·dY·B backward)
// seg_outer  D_a[c, j] = Σ_{m ∈ rows of a} P[m,c]·h[m,j]       (dB_a = s·dYᵀ·h, dA_a = gᵀ·X)
//
// Both stream the big operand P (X or dY) exactly once at full width and keep
// the adapter operands, which are small, in LDS or L2. Work is organised per
// segment, so a workgroup never mixes adapters. Reference semantics:
// training/low_rank.py:26-28 and its autograd backward.
//
// The shrink writes h twice: bf16 rows [M, ldh] for the fused GEMM epilogues,
// and "fragments" for seg_outer: h split into bf16 hi + lo (hi + lo carries
// ~16 significant bits) and stored in the exact per-lane order of the B
// operand of v_mfma_f32_16x16x32_bf16. Fragment blocks cover 32 rows counted
// from each segment's first row (segment s starts at padded row
// pad_start[s] = Σ_{s'<s} roundup(len_s', 32)), so every block belongs to one
// segment; rows past a segment's end inside its last block hold zeros.
//   fragment (block B, j-tile t, part p in {hi, lo}), lane L, element e:
//     h[row = 32·B' + 8·(L/16) + e][j = 16·t + L%16]   (B' = block within segment)
//   stored at u32x4 index ((B·jtiles + t)·2 + p)·64 + L.
#include "mlora_common.h"
#include "mlora_host.h"

#include <mutex>
#include <type_traits>
#include <utility>

namespace mlora {

// Padded-row start of every segment (shared by shrink and seg_outer).
struct PadTable {
  int32_t start[kMaxSeg + 1];
};

static int64_t build_pad(PadTable &pt, const SegTable &st) {
  int64_t p = 0;
  for (int s = 0; s < st.n; ++s) {
    pt.start[s] = (int32_t)p;
    p += (int64_t)(st.off[s + 1] - st.off[s] + 31) / 32 * 32;
  }
  pt.start[st.n] = (int32_t)p;
  return p;
}

// ============================================================== shrink
//
// Workgroup: NW waves x 32 rows of one segment, all r <= 32*RT columns of its
// adapter, k in tiles of 64. Both operands go to LDS with direct-to-LDS loads
// into a ring of ShrinkCfg::STAGES stages (up to STAGES-1 tiles in flight):
//   P tile    [32*NW rows x 128 B], chunk c of row m at slot c ^ swz(m) (the
//             GEMM layout: fragment reads conflict-free);
//   Op tile   layout 0 ([r, K]): [32*RT rows j x 128 B], same swizzle;
//             layout 1 ([K, r]): [64 rows k x 64*RT B] natural, read with the
//             transposing LDS read.
// v_mfma_f32_32x32x16_bf16: rows <- P (m), columns <- Op (j). Lane l of a
// P fragment holds row l%32 and k = 32*(l/32) + 8q + e in substep q; the Op
// fragments use the same k set, so the products pair correctly.

template <int RT, int NW = 4, bool SPLIT = false>
struct ShrinkCfg {
  static constexpr int BMS = 32 * NW;                 // rows per workgroup
  static constexpr int OPROWS = 32 * RT;              // j rows (layout 0) / j columns (layout 1)
  static constexpr int P_BYTES = BMS * 128;           // BMS rows x 64 k
  static constexpr int OP_HALF = OPROWS * 128;        // 32*RT x 64 k of one operand
  // SPLIT: the adapter operand arrives as two bf16 matrices hi + lo (hi = bf16(v),
  // lo = bf16(v - hi): ~16 significant bits of an fp32 master); both tiles sit in
  // the stage and every P fragment is multiplied by each, into one accumulator.
  static constexpr int OP_BYTES = OP_HALF * (SPLIT ? 2 : 1);
  static constexpr int STAGE_BYTES = P_BYTES + OP_BYTES;
  // The shrink streams P, so the rate follows the bytes of P in flight per CU.
  // 4 waves (128 rows): ranks <= 64 take 3 stages (<= 72 KB) so that two
  // workgroups share a CU (measured 20% faster than 4 stages and one workgroup;
  // used for ranks <= 32); larger ranks as many stages as 160 KB allows. 8 waves
  // (256 rows, used for ranks 33-64): 4 stages of 40 KB, one workgroup per CU,
  // 96 KB of P in flight instead of 64 KB (3-7% faster at rank 64; slower at 128).
  // 9 waves (288 rows, ranks <= 128): the row count that puts one tile on each CU when 256-row
  // tiles would leave a few for a second round (65520 rows in four segments: 259 tiles of
  // 256 rows, 230 of 288); 3 stages of 40-52 KB.
  // SPLIT: as many stages (at most 3) as fit.
  static constexpr int STAGES_PLAIN = NW == 8 ? 4 : NW == 9 ? 3 : RT <= 2 ? 3 : RT <= 4 ? 4 : 3;
  static constexpr int STAGES_FIT = 163840 / STAGE_BYTES;
  static constexpr int STAGES = SPLIT ? (STAGES_FIT < 3 ? STAGES_FIT : 3) : STAGES_PLAIN;
  static constexpr int WG_PER_CU = NW >= 8 ? 1 : (RT <= 2 && 2 * STAGES * STAGE_BYTES <= 163840) ? 2 : 1;
  static constexpr int THREADS = 64 * NW;
  static constexpr int P_DMA = P_BYTES / 1024 / NW;    // per wave per tile
  // The operand tile(s) of a stage take OP_BLOCKS 1 KB loads, OP_DMA per wave; when NW does not
  // divide them, the last waves issue loads out of range into a 1 KB dummy block after the
  // stages (no data read; every wave issues the same count, so the vmcnt thresholds hold).
  static constexpr int OP_BLOCKS = OP_BYTES / 1024;
  static constexpr int OP_DMA = (OP_BLOCKS + NW - 1) / NW;  // per wave per tile (layout 0 and 1 alike)
  static constexpr bool OP_DUMMY = OP_DMA * NW != OP_BLOCKS;
  static constexpr int LDS_BYTES = STAGES * STAGE_BYTES + (OP_DUMMY ? 1024 : 0);
  static constexpr int OP_HALF_DMA = OP_HALF / 1024;   // 1 KB loads of one operand tile (whole workgroup)
  static_assert(P_DMA * NW * 1024 == P_BYTES && OP_BLOCKS * 1024 == OP_BYTES, "whole 1 KB loads");
  static_assert(!(SPLIT && OP_DUMMY), "the split operand's two tiles divide over the waves");
  static_assert(STAGES >= 2 && LDS_BYTES <= 163840, "the ring fits the LDS");
  static constexpr int DMA = P_DMA + OP_DMA;
  static constexpr int OPROW_B = OPROWS * 2;          // layout 1: bytes per k row
  static_assert(OP_DMA >= 1 && (STAGES - 2) * DMA < 64, "vmcnt field");
};

struct ShrinkArgs {
  const uint16_t *P;
  uint16_t *Hr;  // bf16 [M, ldh]
  u32x4 *Hf;     // fragments (see above) or null
  const float *row_div;  // per-row divisors of Hr, or null
  int64_t ldp, ldh;
  int32_t M, K;
  int32_t op_layout;  // 0: [r, K]; 1: [K, r]
  int32_t jtiles;     // fragment j-tiles per block
  int32_t tile_start[kMaxSeg + 1];
  PadTable pad;
  AdapterTable op;
  const uint16_t *op_lo[kMaxAdapters];  // SPLIT: the lo parts of the adapter operands
  SegTable seg;
};

template <int RT, int OPL, int NW = 4, bool SPLIT = false>
__global__ __launch_bounds__((ShrinkCfg<RT, NW, SPLIT>::THREADS), (ShrinkCfg<RT, NW, SPLIT>::WG_PER_CU)) void
shrink_kernel(const ShrinkArgs args) {
  using C = ShrinkCfg<RT, NW, SPLIT>;
  constexpr int BMS = C::BMS;
  constexpr int ST = C::STAGES;
  __shared__ u32x4 smem[C::LDS_BYTES / 16];  // the epilogue reuses the stages
  MLORA_LDS char *lds = (MLORA_LDS char *)smem;
  const int tid = threadIdx.x, lane = tid & 63, wave = wave_id();

  // workgroup -> (segment, tile)
  const int bid = blockIdx.x;
  int s = 0;
  while (s + 1 < args.seg.n && args.tile_start[s + 1] <= bid) ++s;
  const int a = args.seg.aid[s];
  const int r = args.op.rank[a];
  const float scale = args.op.scale[a];
  const int rel0 = (bid - args.tile_start[s]) * BMS;  // tile start relative to the segment
  const int m0 = args.seg.off[s] + rel0;
  const int mend = args.seg.off[s + 1];
  const int K = args.K;
  const int nk = (K + 63) / 64;
  const int32_t ldp_b = (int32_t)(args.ldp * 2);
  const __amdgpu_buffer_rsrc_t rop = make_rsrc(args.op.ptr[a], (int64_t)r * K * 2);
  const __amdgpu_buffer_rsrc_t rop_lo = SPLIT ? make_rsrc(args.op_lo[a], (int64_t)r * K * 2) : rop;
  // rows past the segment end fall outside this resource and read as zero
  const __amdgpu_buffer_rsrc_t rp = make_rsrc(args.P + (int64_t)m0 * args.ldp, (int64_t)(mend - m0) * ldp_b);

  // ---- loader offsets. P / layout-0 Op: a 1 KB load fills 8 rows of 128 B;
  // lane L lands at slot L%8 of row L/8 and fetches chunk (L%8) ^ swz(row):
  // two lane patterns by the parity of the 8-row block. Chunks past K read zero
  // through a per-tile mask.
  int32_t p_off[2], p_kc[2];
#pragma unroll
  for (int par = 0; par < 2; ++par) {
    const int c = (lane & 7) ^ (lane >> 3) ^ par;
    p_kc[par] = 8 * c;
    p_off[par] = (lane >> 3) * ldp_b + 16 * c;
  }
  // layout 1: a 1 KB load fills 1024 / OPROW_B k rows; lane L lands at byte 16L
  // of the load: k row (16L) / OPROW_B, chunk (L % CPR) of that row
  constexpr int CPR = C::OPROW_B / 16;
  const int o1_row = lane / CPR, o1_c = lane % CPR;
  const int32_t o1_off = 8 * o1_c < r ? o1_row * r * 2 + 16 * o1_c : kOOB;
  const bool kmask = K % 64 != 0;

  auto issue = [&](auto st_c, int kc) {
    MLORA_LDS char *base = lds + decltype(st_c)::value * C::STAGE_BYTES;
    const int k0 = kc * 64;
    const bool live = kc < nk;
#pragma unroll
    for (int i = 0; i < C::P_DMA; ++i) {
      const int q = wave * C::P_DMA + i;  // 8-row block of the P tile (wave-uniform)
      int32_t off = p_off[q & 1];
      if (!live || (kmask && k0 + p_kc[q & 1] >= K)) off = kOOB;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rp, base + q * 1024, 16, off, 8 * q * ldp_b + 2 * k0, 0, 0);
    }
#pragma unroll
    for (int i = 0; i < C::OP_DMA; ++i) {
      const int qa = wave * C::OP_DMA + i;  // 1 KB block of the stage's operand tiles (wave-uniform)
      const bool dummy = C::OP_DUMMY && qa >= C::OP_BLOCKS;
      MLORA_LDS char *dst = dummy ? lds + ST * C::STAGE_BYTES : base + C::P_BYTES + qa * 1024;
      // SPLIT: blocks past the first operand tile fill the lo tile from the lo matrix
      const bool lo_half = SPLIT && qa >= C::OP_HALF_DMA;
      const int q = lo_half ? qa - C::OP_HALF_DMA : qa;  // block within its operand tile
      const __amdgpu_buffer_rsrc_t rsrc = lo_half ? rop_lo : rop;
      if constexpr (OPL == 0) {
        const int j = 8 * q + (lane >> 3);
        int32_t off = j < r ? p_off[q & 1] - (lane >> 3) * ldp_b + j * K * 2 : kOOB;
        if (!live || dummy || (kmask && k0 + p_kc[q & 1] >= K)) off = kOOB;
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, dst, 16, off, 2 * k0, 0, 0);
      } else {
        const int krow = q * (1024 / C::OPROW_B) + o1_row;  // k row within the tile
        int32_t off = o1_off;
        if (!live || dummy || k0 + krow >= K) off = kOOB;
        // (the scalar offset goes through a variable: written inline in the builtin call,
        // this expression made the host compilation pass drop the kernel instantiation)
        const int32_t soff = (k0 + q * (1024 / C::OPROW_B)) * r * 2;
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, dst, 16, off, soff, 0, 0);
      }
    }
  };

  // ---- fragment addresses (stage-relative)
  const int z = swz(lane & 31);
  int32_t pa[4];  // P: row 32w + l%32, chunk 4h + q
#pragma unroll
  for (int q = 0; q < 4; ++q) pa[q] = (32 * wave + (lane & 31)) * 128 + 16 * ((4 * (lane >> 5) + q) ^ z);
  // layout 0: Op row 32jt + l%32 at the same chunk (add 4096 * jt)
  int32_t oa0[4];
#pragma unroll
  for (int q = 0; q < 4; ++q) oa0[q] = C::P_BYTES + (lane & 31) * 128 + 16 * ((4 * (lane >> 5) + q) ^ z);
  // layout 1: transposing reads; lane i of a 16-lane group points at k row
  // 32h + 8q + (i>>2) (and 4 rows further), columns 32jt + 16g + 4(i&3)
  int32_t oa1[RT];
  {
    const int i = lane & 15, g = (lane >> 4) & 1, h = lane >> 5;
#pragma unroll
    for (int jt = 0; jt < RT; ++jt)
      oa1[jt] = C::P_BYTES + (32 * h + (i >> 2)) * C::OPROW_B + 2 * (32 * jt + 16 * g + 4 * (i & 3));
  }

  f32x16 acc[RT];
#pragma unroll
  for (int j = 0; j < RT; ++j)
#pragma unroll
    for (int v = 0; v < 16; ++v) acc[j][v] = 0.f;

  auto compute = [&](auto st_c) {
    const MLORA_LDS char *base = lds + decltype(st_c)::value * C::STAGE_BYTES;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const bf16x8 pf = as_bf16x8(*(const lds_u4 *)(base + pa[q]));
#pragma unroll
      for (int part = 0; part < (SPLIT ? 2 : 1); ++part) {  // SPLIT: hi tile, then lo tile
        const MLORA_LDS char *ob = base + part * C::OP_HALF;
        bf16x8 of[RT];
        if constexpr (OPL == 0) {
#pragma unroll
          for (int j = 0; j < RT; ++j) of[j] = as_bf16x8(*(const lds_u4 *)(ob + oa0[q] + 4096 * j));
        } else {
          int32_t ad[RT];
#pragma unroll
          for (int j = 0; j < RT; ++j) ad[j] = oa1[j] + 8 * q * C::OPROW_B;
          u32x4 o[RT];
          lds_read_tr16<RT, 4 * C::OPROW_B>(ob, ad, o);
#pragma unroll
          for (int j = 0; j < RT; ++j) of[j] = as_bf16x8(o[j]);
        }
#pragma unroll
        for (int j = 0; j < RT; ++j) acc[j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(pf, of[j], acc[j], 0, 0, 0);
      }
    }
  };

  // ---- pipeline: wait for tile kc, publish it, refill the stage of tile kc-1
  auto step = [&](auto cur, int kc) -> bool {
    if (kc >= nk) return false;
    constexpr int refill = (decltype(cur)::value + ST - 1) % ST;
    wait_vmcnt<(ST - 2) * C::DMA>();
    lds_pipeline_barrier();
    issue(std::integral_constant<int, refill>{}, kc + ST - 1);
    compute(cur);
    return true;
  };
  static_for<ST - 1>([&](auto p) {
    issue(p, decltype(p)::value);
    return true;
  });
  for (int kc = 0; kc < nk; kc += ST) static_for<ST>([&](auto k) { return step(k, kc + decltype(k)::value); });
  wait_vmcnt<0>();
  lds_pipeline_barrier();  // the epilogue reuses the stages as its re-layout buffer

  // ---- epilogue: one 32-wide j tile at a time, each wave re-lays out its 32 rows through its
  // own LDS block (fp32, 16-byte aligned rows of WS floats), then stores the scaled bf16 rows in
  // 16-byte chunks and, if asked, the hi/lo fragments. The acc layout: lane holds j = l%32,
  // m = 8(v/4) + 4(l/32) + v%4.
  constexpr int WS = 36;
  static_assert(NW * 32 * WS * 4 <= ST * C::STAGE_BYTES, "the re-layout blocks fit the stages");
  MLORA_LDS float *wb = (MLORA_LDS float *)lds + wave * 32 * WS;
  const int wrow = m0 + 32 * wave;  // first row of this wave
  const int vrows = min(32, mend - wrow);  // this wave's rows in the segment (<= 0: none)
  // rows past the segment end fall outside rh: their stores are dropped
  const __amdgpu_buffer_rsrc_t rh =
      make_rsrc(args.Hr + (int64_t)(vrows > 0 ? wrow : 0) * args.ldh, (int64_t)max(vrows, 0) * args.ldh * 2);
  // h rows: lane L stores row 16p + L/4, columns 8(L%4) .. +7 of the j tile (pass p = 0, 1)
  const int hr_row = lane >> 2, hr_c8 = 8 * (lane & 3);
  float rdiv[2] = {1.f, 1.f};
  if (args.row_div != nullptr) {
#pragma unroll
    for (int p = 0; p < 2; ++p) {
      const int row = wrow + 16 * p + hr_row;
      if (row < mend) rdiv[p] = args.row_div[row];
    }
  }
  const bool frag = args.Hf != nullptr && wrow < mend;  // a wave past the segment end owns no block
  const int64_t block = (args.pad.start[s] + rel0 + 32 * wave) / 32;
  MLORA_GLOBAL u32x4 *hf = gp(args.Hf);
  auto wave_lds_sync = [] {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  };
#pragma unroll
  for (int j = 0; j < RT; ++j) {
    if (32 * j >= r) break;  // uniform
#pragma unroll
    for (int v = 0; v < 16; ++v) {
      const int ml = 8 * (v >> 2) + 4 * (lane >> 5) + (v & 3);
      wb[ml * WS + (lane & 31)] = acc[j][v] * scale;
    }
    wave_lds_sync();
    if (32 * j + hr_c8 < r) {
#pragma unroll
      for (int p = 0; p < 2; ++p) {
        const int rl = 16 * p + hr_row;
        const MLORA_LDS f32x4 *src = (const MLORA_LDS f32x4 *)(wb + rl * WS + hr_c8);
        const f32x4 x0 = src[0], x1 = src[1];
        float h[8] = {x0[0], x0[1], x0[2], x0[3], x1[0], x1[1], x1[2], x1[3]};
        if (args.row_div != nullptr) {
#pragma unroll
          for (int e = 0; e < 8; ++e) h[e] = h[e] / rdiv[p];
        }
        const u32x4 d = {pack2_bf16(h[0], h[1]), pack2_bf16(h[2], h[3]), pack2_bf16(h[4], h[5]), pack2_bf16(h[6], h[7])};
        buf_store16(rh, (int32_t)((rl * args.ldh + 32 * j + hr_c8) * 2), d);
      }
    }
    if (frag) {
#pragma unroll
      for (int sub = 0; sub < 2; ++sub) {
        const int t = 2 * j + sub;
        if (16 * t < r) {
          float v8[8];
#pragma unroll
          for (int e = 0; e < 8; ++e) v8[e] = wb[(8 * (lane >> 4) + e) * WS + 16 * sub + (lane & 15)];
          u32x4 hi, lo;
          split_hi_lo(v8, hi, lo);
          const int64_t base = ((block * args.jtiles + t) * 2) * 64 + lane;
          hf[base] = hi;
          hf[base + 64] = lo;
        }
      }
    }
    wave_lds_sync();  // every lane has read the block before the next j tile overwrites it
  }
}

template <int RT, int NW = 4, bool SPLIT = false>
static void launch_shrink_rt(const ShrinkArgs &a, int nblocks, hipStream_t stream) {
  constexpr int T = ShrinkCfg<RT, NW, SPLIT>::THREADS;
  if (a.op_layout == 0)
    hipLaunchKernelGGL((shrink_kernel<RT, 0, NW, SPLIT>), dim3(nblocks), dim3(T), 0, stream, a);
  else
    hipLaunchKernelGGL((shrink_kernel<RT, 1, NW, SPLIT>), dim3(nblocks), dim3(T), 0, stream, a);
}

// ============================================================== seg_outer
//
// Work item = (row chunk of one segment, OUT_J-wide j block, OUT_C-wide c block).
// The NWO waves of a workgroup walk the chunk's 32-row steps together, each
// wave owning 64 of the OUT_C = 64·NWO columns, and each item leaves one fp32
// partial [OUT_C c x OUT_J j] (OUT_J = 64, or 128 when most rows have an
// adapter of rank > 64); a second kernel adds an adapter's partials in chunk
// order. Per step the workgroup moves, with direct-to-LDS loads, the P block
// [32 rows x OUT_C c] (2·OUT_C contiguous bytes per row) and the step's h
// fragments (hi and lo, OUT_J j) into one of OUTER_STAGES LDS stages, so the next
// step is in flight while one is multiplied. P stays in its natural layout; the
// gfx950 transposing LDS read (ds_read_b64_tr_b16) turns 4 rows x 4 columns
// into per-column runs of rows, i.e. the A operand of v_mfma_f32_16x16x32_bf16
// (rows <- c, contraction <- the 32 rows of the step, columns <- j). The h
// fragments are stored by the shrink in that MFMA's B-operand order and are
// read as they are (16 bytes per lane).
//
// Column block: every c block of a chunk reads the chunk's h fragments again. The
// items of a chunk run on one XCD, so after the first read they come from its L2.
// 4 waves (256 columns, three workgroups per CU with 64 j) by default; 8 waves
// (512 columns) for 128 j at C <= 4096, where the wider block was faster
// (C = 3072, rank 128: 67 vs 72 us; with 64 j the 4-wave form was faster: C = 1536
// 58.5 vs 63 us, C = 3072 106 vs 111 us).

constexpr int kMaxChunkRows = 32768;
constexpr int kWideOuterMaxC = 4096;  // C up to which the 8-wave (512-column) form runs with 128 j
// Two stages (one step in flight while one is multiplied): 48 KB (4 waves, 64 j) lets three
// workgroups share a CU, measured 7-8% faster than three stages and two workgroups
// (and than more work items, whose partial sums cost more); 80 KB (8 waves) two.
constexpr int OUTER_STAGES = 2;

// NJ: 16-wide j tiles per work item (4: 64 j; 8: 128 j, for adapters of rank 65-128, so that
// P is streamed once per chunk instead of once per 64 j).
template <int NWO, int NJ>
struct OuterCfg {
  static constexpr int OUT_C = 64 * NWO;                          // c per workgroup
  static constexpr int OUT_J = 16 * NJ;                           // j per workgroup
  static constexpr int P_BYTES = 32 * OUT_C * 2;                  // one step of P: 32 rows
  static constexpr int H_BYTES = NJ * 2 * 1024;                   // one step of h: NJ j-tiles x {hi, lo}
  static constexpr int STAGE_BYTES = P_BYTES + H_BYTES;
  static constexpr int PL = P_BYTES / 1024 / NWO;                 // P loads per wave and step
  static constexpr int HL = 2 * NJ / NWO;                         // h loads per wave and step
  static constexpr int DMA = PL + HL;
  static constexpr int CPR = OUT_C / 8;                           // 16-byte chunks per P row
  static constexpr int RPL = 64 / CPR;                            // P rows per 1 KB load
  // waves per SIMD the registers are sized for: 64 j: 3 (4-wave) or 2 (8-wave) workgroups per
  // CU; 128 j (twice the accumulators): two 4-wave or one 8-wave workgroup
  static constexpr int WAVES_PER_EU = NJ == 8 ? 2 : NWO == 8 ? 4 : 2;
  static_assert(PL * NWO * 1024 == P_BYTES && HL * NWO == 2 * NJ, "whole 1 KB loads per wave");
  static_assert(OUTER_STAGES * STAGE_BYTES <= 163840, "the stages fit the LDS");
};

struct OuterArgs {
  const uint16_t *P;
  const u32x4 *Hf;
  float *ws;
  int64_t ldp;
  int32_t M, C;
  int32_t chunk_rows;
  int32_t cblocks, jblocks;  // jblocks = ceil(max rank / 64)
  int32_t rpad;              // 64 * jblocks: partial row length
  int32_t jtiles;            // fragment j-tiles per block
  int32_t chunk_start[kMaxSeg + 1];
  int32_t item_start[kMaxSeg + 1];  // first work item of each segment
  int32_t rank[kMaxAdapters];
  PadTable pad;
  SegTable seg;
};

template <int NWO, int NJ>
__global__ __launch_bounds__((64 * NWO), (OuterCfg<NWO, NJ>::WAVES_PER_EU)) void seg_outer_kernel(const OuterArgs args) {
  using OC = OuterCfg<NWO, NJ>;
  constexpr int OUT_C = OC::OUT_C;
  __shared__ u32x4 smem[OUTER_STAGES * OC::STAGE_BYTES / 16];
  MLORA_LDS char *lds = (MLORA_LDS char *)smem;
  const int tid = threadIdx.x, lane = tid & 63, wave = wave_id();
  // Work items: per segment with an adapter, its chunks x its j blocks (ceil(r / OUT_J), so no
  // item is empty) x the c blocks, c fastest. The items of one chunk are consecutive logical ids,
  // and these run on one XCD, whose L2 then serves the chunk's h fragments to all of them.
  const int item = xcd_contiguous(blockIdx.x, gridDim.x);
  int s = 0;
  while (s + 1 < args.seg.n && args.item_start[s + 1] <= item) ++s;
  const int a = args.seg.aid[s];
  const int r = args.rank[a];
  const int local = item - args.item_start[s];
  const int jbs = (r + OC::OUT_J - 1) / OC::OUT_J;
  const int cb = local % args.cblocks;
  const int jb = (local / args.cblocks) % jbs;
  const int chunk = args.chunk_start[s] + local / (args.cblocks * jbs);
  const int j0 = jb * OC::OUT_J;
  const int rel0 = (chunk - args.chunk_start[s]) * args.chunk_rows;  // multiple of 32
  const int row0 = args.seg.off[s] + rel0;
  const int rend = min(row0 + args.chunk_rows, args.seg.off[s + 1]);
  const int nsteps = (rend - row0 + 31) / 32;
  const int64_t block0 = (args.pad.start[s] + rel0) / 32;
  const int c0 = cb * OUT_C;
  const int32_t ldp_b = (int32_t)(args.ldp * 2);
  // P rows past the chunk end fall outside rp and read as zero
  const __amdgpu_buffer_rsrc_t rp =
      make_rsrc(args.P + (int64_t)row0 * args.ldp + c0, (int64_t)(rend - row0) * ldp_b);
  const __amdgpu_buffer_rsrc_t rh =
      make_rsrc(args.Hf + (block0 * args.jtiles) * 128, (int64_t)nsteps * args.jtiles * 2048);

  // Loader. A 1 KB P load covers RPL rows of CPR 16-byte chunks; chunk cc of
  // step row rr sits at LDS slot cc ^ (4 * (rr & 3)), so lane L fetches the
  // chunk whose slot it fills. This wave's loads: P loads PL·w .. PL·w + PL - 1
  // of the step, h loads HL·w .. HL·w + HL - 1 of the 8.
  int32_t p_off[OC::PL], p_row[OC::PL];
#pragma unroll
  for (int i = 0; i < OC::PL; ++i) {
    const int q = OC::PL * wave + i;
    const int row = OC::RPL * q + lane / OC::CPR;
    const int cc = (lane % OC::CPR) ^ (4 * (row & 3));
    p_off[i] = c0 + 8 * cc < args.C ? (lane / OC::CPR) * ldp_b + 16 * cc : kOOB;
    p_row[i] = OC::RPL * q;
  }
  const int32_t h_step = args.jtiles * 2048;
  auto issue = [&](auto st_c, int step) {
    MLORA_LDS char *base = lds + decltype(st_c)::value * OC::STAGE_BYTES;
    const bool live = step < nsteps;
#pragma unroll
    for (int i = 0; i < OC::PL; ++i) {
      const int q = OC::PL * wave + i;  // wave-uniform
      const int32_t off = live ? p_off[i] : kOOB;
      // (operands go through variables: template-dependent expressions written inline in the
      // builtin call make the host compilation pass drop the kernel instantiation)
      const int32_t soff = (32 * step + p_row[i]) * ldp_b;
      MLORA_LDS void *dst = base + q * 1024;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rp, dst, 16, off, soff, 0, 0);
    }
#pragma unroll
    for (int i = 0; i < OC::HL; ++i) {
      const int q = OC::HL * wave + i;  // (j-tile, part) = (q / 2, q % 2) of this j block
      const int t = (j0 >> 4) + (q >> 1);
      const int32_t off = live && 16 * t < r ? ((t * 2 + (q & 1)) * 64 + lane) * 16 : kOOB;
      const int32_t soff = step * h_step;
      MLORA_LDS void *dst = base + OC::P_BYTES + q * 1024;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rh, dst, 16, off, soff, 0, 0);
    }
  };

  // Fragment addresses (stage-relative). A operand of c tile t (16 columns):
  // lane i of a 16-lane group reads rows 8g + (i>>2) (+4) and the 4 columns at
  // 16t + 4(i&3) of this wave's 64; the transposing read hands lane j column
  // 16t + j, rows 8g..8g+3: 4 of the 8 rows the MFMA wants from lane 16g + j.
  const int li = lane & 15, lg = lane >> 4;
  int32_t a_addr[4];
#pragma unroll
  for (int t = 0; t < 4; ++t) {
    const int row = 8 * lg + (li >> 2);
    const int cc = 8 * wave + 2 * t + ((li & 3) >> 1);
    a_addr[t] = row * (OUT_C * 2) + 16 * (cc ^ (4 * (row & 3))) + 8 * (li & 1);
  }

  f32x4 acc[4][NJ];
#pragma unroll
  for (int t = 0; t < 4; ++t)
#pragma unroll
    for (int q = 0; q < NJ; ++q) acc[t][q] = f32x4{0.f, 0.f, 0.f, 0.f};

  auto compute = [&](auto st_c) {
    const MLORA_LDS char *base = lds + decltype(st_c)::value * OC::STAGE_BYTES;
    bf16x8 hi[NJ], lo[NJ], af[4];
#pragma unroll
    for (int q = 0; q < NJ; ++q) {
      hi[q] = as_bf16x8(*(const lds_u4 *)(base + OC::P_BYTES + (2 * q) * 1024 + 16 * lane));
      lo[q] = as_bf16x8(*(const lds_u4 *)(base + OC::P_BYTES + (2 * q + 1) * 1024 + 16 * lane));
    }
    u32x4 at[4];
    lds_read_tr16_x4<4 * OUT_C * 2>(base, a_addr, at);  // rows +4: the second half of each fragment
#pragma unroll
    for (int t = 0; t < 4; ++t) af[t] = as_bf16x8(at[t]);
#pragma unroll
    for (int t = 0; t < 4; ++t)
#pragma unroll
      for (int q = 0; q < NJ; ++q) {
        acc[t][q] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af[t], hi[q], acc[t][q], 0, 0, 0);
        acc[t][q] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af[t], lo[q], acc[t][q], 0, 0, 0);
      }
  };

  // OUTER_STAGES-deep pipeline, one barrier per step: wait for step i, make it
  // visible, refill the stage step i-1 used (every wave is past it), multiply.
  // Loads past the last step carry no data but keep the wait counts uniform.
  // The loop is unrolled by the stage count so that every stage offset is a
  // constant: with run-time stage indices the compiler cannot tell the loads
  // in flight from the stage being read and waits for all of them.
  auto step = [&](auto cur, int i) -> bool {
    if (i >= nsteps) return false;
    constexpr int refill = (decltype(cur)::value + OUTER_STAGES - 1) % OUTER_STAGES;
    wait_vmcnt<(OUTER_STAGES - 2) * OC::DMA>();  // this wave's loads of step i landed
    lds_pipeline_barrier();                        // everyone's did; everyone is done with step i-1
    issue(std::integral_constant<int, refill>{}, i + OUTER_STAGES - 1);
    compute(cur);
    return true;
  };
  static_for<OUTER_STAGES - 1>([&](auto p) {
    issue(p, decltype(p)::value);
    return true;
  });
  for (int i = 0; i < nsteps; i += OUTER_STAGES)
    static_for<OUTER_STAGES>([&](auto k) { return step(k, i + decltype(k)::value); });
  wait_vmcnt<0>();  // nothing may still write LDS when the workgroup ends

  // partial layout: ws[chunk][c][rpad]; lane holds c = c0 + 64w + 16t + 4(l/16) + v, j = j0 + 16q + l%16
  MLORA_GLOBAL float *dst = gp(args.ws) + (int64_t)chunk * args.C * args.rpad;
#pragma unroll
  for (int t = 0; t < 4; ++t)
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const int c = c0 + 64 * wave + 16 * t + 4 * lg + v;
      if (c >= args.C) continue;
#pragma unroll
      for (int q = 0; q < NJ; ++q) {
        const int j = j0 + 16 * q + li;
        if (j < r) dst[(int64_t)c * args.rpad + j] = acc[t][q][v];
      }
    }
}

struct ReduceArgs {
  const float *ws;
  int64_t C;
  int32_t rpad;
  int32_t out_layout, out_dtype;
  int32_t n_adapters;
  int32_t chunk_start[kMaxSeg + 1];
  int32_t rank[kMaxAdapters];
  void *out[kMaxAdapters];
  SegTable seg;
};

// One thread per (adapter, c, 4 consecutive j): partials summed in chunk order
// (deterministic). The 16-byte loads of up to RB chunks are issued together and
// then added in order, so a thread waits for a batch of loads, not for each.
__global__ __launch_bounds__(256) void seg_outer_reduce_kernel(const ReduceArgs args) {
  constexpr int RB = 8;
  const int a = blockIdx.y;
  const int r = args.rank[a];
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;  // (c, j/4)
  const int rq = r / 4;                                          // r is a multiple of 8
  if (r == 0 || args.out[a] == nullptr || idx >= args.C * rq) return;
  const int64_t c = idx / rq;
  const int j = 4 * (int)(idx % rq);
  const int64_t pitch = args.C * args.rpad;  // floats between the partials of consecutive chunks
  const MLORA_GLOBAL float *base = gp(args.ws) + c * args.rpad + j;
  f32x4 sum = {0.f, 0.f, 0.f, 0.f};
  for (int s = 0; s < args.seg.n; ++s) {
    if (args.seg.aid[s] != a) continue;
    const int ch1 = args.chunk_start[s + 1];
    for (int ch = args.chunk_start[s]; ch < ch1; ch += RB) {
      f32x4 v[RB];
#pragma unroll
      for (int u = 0; u < RB; ++u)
        v[u] = ch + u < ch1 ? *(const MLORA_GLOBAL f32x4 *)(base + (int64_t)(ch + u) * pitch) : f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int u = 0; u < RB; ++u)
        if (ch + u < ch1) sum += v[u];
    }
  }
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const int64_t o = args.out_layout == 0 ? c * r + j + e : (int64_t)(j + e) * args.C + c;
    if (args.out_dtype == MLORA_F32)
      gp(static_cast<float *>(args.out[a]))[o] = sum[e];
    else
      gp(static_cast<uint16_t *>(args.out[a]))[o] = f32_to_bf16_rne(sum[e]);
  }
}

// Chunking shared by the entry point and the workspace query.
struct OuterPlan {
  int32_t nwo = 4;  // waves per workgroup: 64·nwo columns per work item
  int32_t nj = 4;   // 16-wide j tiles per work item
  int32_t chunk_rows = 0, cblocks = 0, jblocks = 0, rpad = 0, n_chunks = 0;
  int64_t n_items = 0;
  int32_t chunk_start[kMaxSeg + 1];
  int64_t item_start[kMaxSeg + 1];
};

static void plan_outer(OuterPlan &pl, const SegTable &st, const int32_t *rank, int64_t C) {
  int rmax = 0;
  int64_t rows = 0, rows_wide = 0;  // rows with an adapter; of them, rows of rank > 64
  for (int s = 0; s < st.n; ++s) {
    const int a = st.aid[s];
    const int len = st.off[s + 1] - st.off[s];
    if (a >= 0 && rank[a] > 0 && len > 0) {
      rows += len;
      if (rank[a] > 64) rows_wide += len;
      rmax = rank[a] > rmax ? rank[a] : rmax;
    }
  }
  // 128 j per item when most rows have an adapter of rank > 64 (their P is then streamed once
  // instead of twice); with few such rows the 64-j items, whose second j block exits at once
  // for the smaller ranks, are faster (config 4's mixed ranks: 3%)
  pl.nj = 2 * rows_wide > rows ? 8 : 4;
  const int out_j = 16 * pl.nj;
  pl.nwo = C <= kWideOuterMaxC && pl.nj == 8 ? 8 : 4;
  const int64_t out_c = 64 * (int64_t)pl.nwo;
  pl.cblocks = (int32_t)((C + out_c - 1) / out_c);
  pl.jblocks = (rmax + out_j - 1) / out_j;
  pl.rpad = pl.jblocks * out_j;
  // Chunk rows: the candidate (a multiple of 64 from 256 rows) of least modelled time. The model,
  // calibrated on MI355X at the Wan / FLUX shapes: a work item moves cr·(2·OUT_C + 4·OUT_J) bytes
  // of P and h fragments and writes its OUT_C x OUT_J partial sums; a CU running k items at once
  // streams about 24 / 38 / 50 KB per us (k = 1 / 2 / 3), the chip about 5.8 MB per us; the
  // fragments come from HBM once (the items of a chunk share an XCD's L2); the reduction reads
  // the partial sums once more. A plan whose items exceed the CUs' slots pays a whole extra
  // round, so the model favours chunks that give every item a slot.
  const int w = pl.nj == 8 ? (pl.nwo == 8 ? 1 : 2) : (pl.nwo == 8 ? 2 : 3);  // workgroups per CU
  constexpr double kRate[4] = {0.0, 24e3, 38e3, 50e3};  // bytes per us per CU, k workgroups
  constexpr double kChip = 5.8e6;                       // bytes per us
  constexpr int kCUs = 256;
  int64_t max_len = 0, frag = 0;
  for (int s = 0; s < st.n; ++s) {
    const int a = st.aid[s];
    const int64_t len = st.off[s + 1] - st.off[s];
    if (a >= 0 && rank[a] > 0 && len > 0) {
      max_len = len > max_len ? len : max_len;
      frag += (len + 31) / 32 * 32 * ((rank[a] + 15) / 16 * 16) * 4;
    }
  }
  int64_t best_cr = 512;
  double best_t = -1.0;
  const int64_t cr_hi = max_len < kMaxChunkRows ? (max_len + 63) / 64 * 64 : kMaxChunkRows;
  for (int64_t cr = 256; cr <= (cr_hi > 256 ? cr_hi : 256); cr += 64) {
    int64_t items = 0, nch = 0;
    for (int s = 0; s < st.n; ++s) {
      const int a = st.aid[s];
      const int64_t len = st.off[s + 1] - st.off[s];
      if (a >= 0 && rank[a] > 0 && len > 0) {
        const int64_t c = (len + cr - 1) / cr;
        nch += c;
        items += c * pl.cblocks * ((rank[a] + out_j - 1) / out_j);
      }
    }
    const double part = (double)nch * C * pl.rpad * 4;
    const double total = (double)rows * C * 2 + (double)frag + part;
    const double rows_item = (double)(cr < max_len ? cr : max_len);
    const double item_b = rows_item * (2.0 * out_c + 4.0 * out_j) + 4.0 * out_c * out_j;
    double t_cu;
    if (items <= (int64_t)kCUs * w) {
      const int k = (int)((items + kCUs - 1) / kCUs);
      t_cu = item_b * k / kRate[k < 1 ? 1 : k];
    } else {
      const int64_t rounds = (items + (int64_t)kCUs * w - 1) / ((int64_t)kCUs * w);
      t_cu = (double)rounds * item_b * w / kRate[w];
    }
    const double t = (total / kChip > t_cu ? total / kChip : t_cu) + part / kChip;
    if (best_t < 0.0 || t < best_t) {
      best_t = t;
      best_cr = cr;
    }
  }
  pl.chunk_rows = (int32_t)best_cr;
  int32_t n = 0;
  int64_t items = 0;
  for (int s = 0; s < st.n; ++s) {
    pl.chunk_start[s] = n;
    pl.item_start[s] = items;
    const int a = st.aid[s];
    const int len = st.off[s + 1] - st.off[s];
    if (a >= 0 && rank[a] > 0 && len > 0) {
      const int c = (len + pl.chunk_rows - 1) / pl.chunk_rows;
      n += c;
      items += (int64_t)c * pl.cblocks * ((rank[a] + out_j - 1) / out_j);
    }
  }
  pl.chunk_start[st.n] = n;
  pl.item_start[st.n] = items;
  pl.n_chunks = n;
  pl.n_items = items;
}

static int64_t frag_bytes(const SegTable &st, int jtiles) {
  PadTable pt;
  return build_pad(pt, st) / 32 * jtiles * 2048;
}

}  // namespace mlora

using namespace mlora;

extern "C" int64_t mlora_frag_bytes(int64_t M, int32_t frag_jtiles, const int64_t *seg_offsets,
                                    const int32_t *adapter_ids, int32_t n_segments) {
  SegTable st;
  int s = build_segtable(st, M, seg_offsets, adapter_ids, n_segments, kMaxAdapters);
  if (s) return s;
  if (frag_jtiles < 0 || frag_jtiles > kMaxRank / 16) return MLORA_ERR_INVALID;
  return frag_bytes(st, frag_jtiles);
}

extern "C" int mlora_shrink(const void *p, int64_t ldp, int64_t M, int64_t K, const void *const *op_ptrs,
                            const void *const *op_lo_ptrs, int op_layout, const int32_t *ranks, const float *scales,
                            int32_t n_adapters, const int64_t *seg_offsets, const int32_t *adapter_ids,
                            int32_t n_segments, void *h_rows, int64_t ldh, void *h_frag, int32_t frag_jtiles,
                            const float *row_div, void *stream) {
  ShrinkArgs a{};
  int st = build_segtable(a.seg, M, seg_offsets, adapter_ids, n_segments, n_adapters);
  if (st) return st;
  if ((st = build_adapters(a.op, a.seg, op_ptrs, ranks, scales, n_adapters))) return st;
  if (op_layout != 0 && op_layout != 1) return MLORA_ERR_INVALID;
  if (K < 0 || K > INT32_MAX - 1024) return MLORA_ERR_INVALID;
  const bool split = op_lo_ptrs != nullptr;
  for (int i = 0; i < kMaxAdapters; ++i) a.op_lo[i] = nullptr;
  if (split) {  // every used operand needs its lo part, aligned like the hi part
    for (int i = 0; i < n_adapters; ++i) {
      if (a.op.ptr[i] == nullptr) continue;
      if (op_lo_ptrs[i] == nullptr) return MLORA_ERR_INVALID;
      if (!aligned16(op_lo_ptrs[i])) return MLORA_ERR_UNSUPPORTED;
      a.op_lo[i] = static_cast<const uint16_t *>(op_lo_ptrs[i]);
    }
  }
  const int rmax = max_used_rank(a.seg, a.op);
  if (rmax == 0 || M == 0) return MLORA_OK;
  if ((st = check_bf16_matrix(p, ldp, M, K))) return st;
  if ((st = check_bf16_matrix(h_rows, ldh, M, rmax))) return st;
  // 31-bit byte offsets inside the buffer resources of one tile / one operand / 32 h rows
  if (ldp * 2 * 256 >= kOOB || K * 2 * (int64_t)kMaxRank >= kOOB || ldh * 2 * 32 >= kOOB) return MLORA_ERR_LIMIT;
  if (h_frag != nullptr) {
    if (frag_jtiles * 16 < rmax || frag_jtiles > kMaxRank / 16) return MLORA_ERR_INVALID;
    if (!aligned16(h_frag)) return MLORA_ERR_UNSUPPORTED;
  }
  a.P = static_cast<const uint16_t *>(p);
  a.Hr = static_cast<uint16_t *>(h_rows);
  a.Hf = static_cast<u32x4 *>(h_frag);
  a.row_div = row_div;
  a.ldp = ldp;
  a.ldh = ldh;
  a.M = (int32_t)M;
  a.K = (int32_t)K;
  a.op_layout = op_layout;
  a.jtiles = frag_jtiles;
  build_pad(a.pad, a.seg);
  hipStream_t s = static_cast<hipStream_t>(stream);
  // tiles of every segment with an adapter of rank > 0 (tile_rows rows each); false: no tile
  auto plan_tiles = [](ShrinkArgs &b, int tile_rows, int64_t &n) {
    n = 0;
    for (int sg = 0; sg < b.seg.n; ++sg) {
      b.tile_start[sg] = (int32_t)n;
      const int ad = b.seg.aid[sg];
      const int len = b.seg.off[sg + 1] - b.seg.off[sg];
      if (ad >= 0 && b.op.rank[ad] > 0 && len > 0) n += (len + tile_rows - 1) / tile_rows;
    }
    b.tile_start[b.seg.n] = (int32_t)n;
    return n > 0;
  };
  const int rt = (rmax + 31) / 32;
  int64_t n = 0;
  if (split && op_layout == 0 && rt > 4) {
    // fp32 masters [r, K] of rank > 128: two passes of the 128-column kernel, columns [0, 128)
    // and [128, r) (operand rows 128.., h columns 128.., fragment j-tiles 8..). One pass over
    // all columns would hold the P tile and both 256-row operand tiles in every stage (80 KB:
    // two stages only), and measured 6-11x slower than the two passes.
    ShrinkArgs hi_cols = a;
    for (int i = 0; i < n_adapters; ++i) {
      a.op.rank[i] = a.op.rank[i] < 128 ? a.op.rank[i] : 128;
      const bool more = hi_cols.op.rank[i] > 128;
      hi_cols.op.rank[i] = more ? hi_cols.op.rank[i] - 128 : 0;
      hi_cols.op.ptr[i] = more ? hi_cols.op.ptr[i] + (int64_t)128 * K : nullptr;
      hi_cols.op_lo[i] = more ? hi_cols.op_lo[i] + (int64_t)128 * K : nullptr;
    }
    hi_cols.Hr = a.Hr + 128;
    hi_cols.Hf = a.Hf != nullptr ? a.Hf + 8 * 2 * 64 : nullptr;
    if (plan_tiles(a, 128, n)) hipLaunchKernelGGL((shrink_kernel<4, 0, 4, true>), dim3((int)n), dim3(256), 0, s, a);
    if (plan_tiles(hi_cols, 128, n))
      hipLaunchKernelGGL((shrink_kernel<4, 0, 4, true>), dim3((int)n), dim3(256), 0, s, hi_cols);
    return launch_status();
  }
  // ranks 33-64: 256-row workgroups of 8 waves (more of P in flight per CU)
  if (!plan_tiles(a, rt == 2 ? ShrinkCfg<2, 8>::BMS : 128, n)) return MLORA_OK;
  if (!split && rt <= 4) {
    // 288-row workgroups of 9 waves when they give every CU at most one tile and the default
    // tiles would not: cost = rounds x rows a CU takes per round (256 CUs; the 4-wave tiles of
    // ranks <= 32 run two workgroups per CU). At ranks <= 64 a tile's time hardly depends on its
    // rows (its k-steps stream at a latency-bound pace): 65520 rows in four segments take 259
    // tiles of 256 rows (two rounds) or 230 of 288 (one), and the shrink 47 instead of 67 us at
    // K = 1536. At ranks 65-128 the rows do set a tile's time (256-row tiles of 8 waves, in two
    // rounds instead of three of 128 rows, measured 3-12% slower at 16 x 4608 rows), so the
    // 288-row tiles are taken only where they save rows per CU: 16 x 4608 rows are 576 tiles of
    // 128 rows (three rounds, 384 rows per CU) or 256 of 288 (one round, 288 rows per CU).
    constexpr int64_t kCUs = 256;
    const int64_t wg = rt <= 1 ? 2 : 1, rows = rt == 2 ? 256 : 128;
    const int64_t cost_default = (n + kCUs * wg - 1) / (kCUs * wg) * rows * wg;
    int64_t n9 = 0;
    plan_tiles(a, ShrinkCfg<2, 9>::BMS, n9);
    const int64_t cost9 = (n9 + kCUs - 1) / kCUs * ShrinkCfg<2, 9>::BMS;
    if (cost9 < cost_default) {
      if (rt <= 1) launch_shrink_rt<1, 9>(a, (int)n9, s);
      else if (rt == 2) launch_shrink_rt<2, 9>(a, (int)n9, s);
      else launch_shrink_rt<4, 9>(a, (int)n9, s);
      return launch_status();
    }
    plan_tiles(a, rows, n);
  }
  if (split) {
    // fp32 masters: the same tile shapes with both operand parts in each stage
    if (rt <= 1) launch_shrink_rt<1, 4, true>(a, (int)n, s);
    else if (rt == 2) launch_shrink_rt<2, 8, true>(a, (int)n, s);
    else if (rt <= 4) launch_shrink_rt<4, 4, true>(a, (int)n, s);
    else hipLaunchKernelGGL((shrink_kernel<8, 1, 4, true>), dim3((int)n), dim3(256), 0, s, a);  // layout 1
    return launch_status();
  }
  if (rt <= 1) launch_shrink_rt<1>(a, (int)n, s);
  else if (rt == 2) launch_shrink_rt<2, 8>(a, (int)n, s);
  else if (rt <= 4) launch_shrink_rt<4>(a, (int)n, s);
  // ranks up to 192 in layout 0 (the stacked A of three linears that read one input):
  // six 32-column tiles instead of eight (layout 1 needs 1 KB loads of whole k rows)
  else if (rt <= 6 && a.op_layout == 0)
    hipLaunchKernelGGL((shrink_kernel<6, 0>), dim3((int)n), dim3(256), 0, s, a);
  else launch_shrink_rt<8>(a, (int)n, s);
  return launch_status();
}

static int outer_setup(OuterArgs &a, OuterPlan &pl, int64_t M, int64_t C, const int32_t *ranks, int32_t n_adapters,
                       const int64_t *seg_offsets, const int32_t *adapter_ids, int32_t n_segments) {
  int st = build_segtable(a.seg, M, seg_offsets, adapter_ids, n_segments, n_adapters);
  if (st) return st;
  if (n_adapters < 0) return MLORA_ERR_INVALID;
  if (n_adapters > kMaxAdapters) return MLORA_ERR_LIMIT;
  if (n_adapters > 0 && ranks == nullptr) return MLORA_ERR_INVALID;
  if (C < 0 || C > INT32_MAX - 1024) return MLORA_ERR_INVALID;
  for (int i = 0; i < kMaxAdapters; ++i) a.rank[i] = 0;
  for (int i = 0; i < n_adapters; ++i) {
    if (ranks[i] < 0 || (ranks[i] > 0 && ranks[i] < 8) || ranks[i] % 8) return MLORA_ERR_INVALID;
    if (ranks[i] > kMaxRank) return MLORA_ERR_LIMIT;
    a.rank[i] = ranks[i];
  }
  plan_outer(pl, a.seg, a.rank, C);
  return MLORA_OK;
}

extern "C" int64_t mlora_seg_outer_workspace_bytes(int64_t M, int64_t C, const int32_t *ranks, int32_t n_adapters,
                                                   const int64_t *seg_offsets, const int32_t *adapter_ids,
                                                   int32_t n_segments) {
  OuterArgs a{};
  OuterPlan pl;
  int st = outer_setup(a, pl, M, C, ranks, n_adapters, seg_offsets, adapter_ids, n_segments);
  if (st) return st;
  return (int64_t)pl.n_chunks * C * pl.rpad * (int64_t)sizeof(float);
}

// Validation and launches shared by mlora_seg_outer and mlora_seg_outer_noalloc; a and pl
// come from outer_setup.
static int seg_outer_run(OuterArgs &a, const OuterPlan &pl, const void *p, int64_t ldp, int64_t M, int64_t C,
                         const void *h_frag, int32_t frag_jtiles, void *const *out_ptrs, int out_layout, int out_dtype,
                         int32_t n_adapters, void *workspace, int64_t workspace_bytes, hipStream_t s) {
  int st;
  if (out_layout != 0 && out_layout != 1) return MLORA_ERR_INVALID;
  if (out_dtype != MLORA_F32 && out_dtype != MLORA_BF16) return MLORA_ERR_UNSUPPORTED;
  if (n_adapters > 0 && out_ptrs == nullptr) return MLORA_ERR_INVALID;
  for (int i = 0; i < n_adapters; ++i)
    if (a.rank[i] > 0 && C > 0 && out_ptrs[i] == nullptr) return MLORA_ERR_INVALID;
  if (C == 0 || n_adapters == 0) return MLORA_OK;
  const int64_t need = (int64_t)pl.n_chunks * C * pl.rpad * (int64_t)sizeof(float);
  if (pl.n_chunks > 0) {
    if ((st = check_bf16_matrix(p, ldp, M, C))) return st;
    if (h_frag == nullptr || !aligned16(h_frag)) return MLORA_ERR_INVALID;
    if (frag_jtiles < 1 || frag_jtiles > kMaxRank / 16) return MLORA_ERR_INVALID;
    for (int i = 0; i < n_adapters; ++i)
      if (a.rank[i] > frag_jtiles * 16) return MLORA_ERR_INVALID;
    if (workspace == nullptr || workspace_bytes < need) return MLORA_ERR_WORKSPACE;
    if (!aligned16(workspace)) return MLORA_ERR_UNSUPPORTED;
    if (ldp * 2 * kMaxChunkRows >= kOOB || (int64_t)(kMaxChunkRows / 32) * frag_jtiles * 2048 >= kOOB)
      return MLORA_ERR_LIMIT;
    a.P = static_cast<const uint16_t *>(p);
    a.Hf = static_cast<const u32x4 *>(h_frag);
    a.ws = static_cast<float *>(workspace);
    a.ldp = ldp;
    a.M = (int32_t)M;
    a.C = (int32_t)C;
    a.chunk_rows = pl.chunk_rows;
    a.cblocks = pl.cblocks;
    a.jblocks = pl.jblocks;
    a.rpad = pl.rpad;
    a.jtiles = frag_jtiles;
    build_pad(a.pad, a.seg);
    const int64_t items = pl.n_items;
    if (items > INT32_MAX) return MLORA_ERR_LIMIT;
    for (int i = 0; i <= a.seg.n; ++i) {
      a.chunk_start[i] = pl.chunk_start[i];
      a.item_start[i] = (int32_t)pl.item_start[i];
    }
    if (pl.nwo == 8 && pl.nj == 8)
      hipLaunchKernelGGL((seg_outer_kernel<8, 8>), dim3((unsigned)items), dim3(512), 0, s, a);
    else if (pl.nwo == 8)
      hipLaunchKernelGGL((seg_outer_kernel<8, 4>), dim3((unsigned)items), dim3(512), 0, s, a);
    else if (pl.nj == 8)
      hipLaunchKernelGGL((seg_outer_kernel<4, 8>), dim3((unsigned)items), dim3(256), 0, s, a);
    else
      hipLaunchKernelGGL((seg_outer_kernel<4, 4>), dim3((unsigned)items), dim3(256), 0, s, a);
    if ((st = launch_status())) return st;
  }
  ReduceArgs ra{};
  ra.ws = static_cast<const float *>(workspace);
  ra.C = C;
  ra.rpad = pl.rpad;
  ra.out_layout = out_layout;
  ra.out_dtype = out_dtype;
  ra.n_adapters = n_adapters;
  ra.seg = a.seg;
  int rmax = 0;
  for (int i = 0; i <= a.seg.n; ++i) ra.chunk_start[i] = pl.chunk_start[i];
  for (int i = 0; i < kMaxAdapters; ++i) {
    ra.rank[i] = i < n_adapters ? a.rank[i] : 0;
    ra.out[i] = i < n_adapters ? out_ptrs[i] : nullptr;
    rmax = ra.rank[i] > rmax ? ra.rank[i] : rmax;
  }
  if (rmax == 0) return MLORA_OK;
  const int64_t blocks_x = (C * (rmax / 4) + 255) / 256;
  if (blocks_x > INT32_MAX) return MLORA_ERR_LIMIT;
  hipLaunchKernelGGL(seg_outer_reduce_kernel, dim3((unsigned)blocks_x, (unsigned)n_adapters), dim3(256), 0, s, ra);
  return launch_status();
}

extern "C" int mlora_seg_outer(const void *p, int64_t ldp, int64_t M, int64_t C, const void *h_frag,
                               int32_t frag_jtiles, void *const *out_ptrs, int out_layout, int out_dtype,
                               const int32_t *ranks, int32_t n_adapters, const int64_t *seg_offsets,
                               const int32_t *adapter_ids, int32_t n_segments, void *workspace,
                               int64_t workspace_bytes, void *stream) {
  OuterArgs a{};
  OuterPlan pl;
  int st = outer_setup(a, pl, M, C, ranks, n_adapters, seg_offsets, adapter_ids, n_segments);
  if (st) return st;
  return seg_outer_run(a, pl, p, ldp, M, C, h_frag, frag_jtiles, out_ptrs, out_layout, out_dtype, n_adapters,
                       workspace, workspace_bytes, static_cast<hipStream_t>(stream));
}

// ---------------------------------------------------------------- seg_outer without allocation
//
// The partial sums of mlora_seg_outer_noalloc live in this file-scope device array
// (one instance per GPU, created when the library's code object is loaded on that
// GPU and held until the process ends). Host code never passes `scratch` itself to a
// kernel (on the host it is a stand-in symbol, not a device address): its device
// address is looked up once per device with hipGetSymbolAddress and kept in
// scratch_address.
namespace mlora {

static __device__ __align__(256) float scratch[MLORA_NOALLOC_SCRATCH_BYTES / sizeof(float)];

constexpr int kMaxDevices = 64;

// Device address of this GPU's scratch array (the current device), looked up on the
// first call per device; MLORA_ERR_DEVICE if there is no current device or the lookup fails.
static int scratch_address(void **out) {
  static std::mutex mu;
  static void *table[kMaxDevices] = {};
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return MLORA_ERR_DEVICE;
  std::lock_guard<std::mutex> lock(mu);
  if (table[dev] == nullptr) {
    void *p = nullptr;
    if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess || p == nullptr) return MLORA_ERR_DEVICE;
    table[dev] = p;
  }
  *out = table[dev];
  return MLORA_OK;
}

}  // namespace mlora

extern "C" int mlora_seg_outer_noalloc(const void *p, int64_t ldp, int64_t M, int64_t C, const void *h_frag,
                                       int32_t frag_jtiles, void *const *out_ptrs, int out_layout, int out_dtype,
                                       const int32_t *ranks, int32_t n_adapters, const int64_t *seg_offsets,
                                       const int32_t *adapter_ids, int32_t n_segments, void *stream) {
  OuterArgs a{};
  OuterPlan pl;
  int st = outer_setup(a, pl, M, C, ranks, n_adapters, seg_offsets, adapter_ids, n_segments);
  if (st) return st;
  if (out_layout != 0 && out_layout != 1) return MLORA_ERR_INVALID;
  if (out_dtype != MLORA_F32 && out_dtype != MLORA_BF16) return MLORA_ERR_UNSUPPORTED;
  if (n_adapters > 0 && out_ptrs == nullptr) return MLORA_ERR_INVALID;
  if (C == 0 || n_adapters == 0) return MLORA_OK;
  // mlora_seg_outer's plan (so the result is the same bit for bit) if its partial sums fit
  const int64_t need = (int64_t)pl.n_chunks * C * pl.rpad * (int64_t)sizeof(float);
  if (need > (int64_t)MLORA_NOALLOC_SCRATCH_BYTES) return MLORA_ERR_LIMIT;
  void *ws = nullptr;
  if ((st = scratch_address(&ws))) return st;
  return seg_outer_run(a, pl, p, ldp, M, C, h_frag, frag_jtiles, out_ptrs, out_layout, out_dtype, n_adapters, ws,
                       MLORA_NOALLOC_SCRATCH_BYTES, static_cast<hipStream_t>(stream));
}

extern "C" int mlora_abi_version(void) { return MLORA_ABI_VERSION; }

#ifndef MLORA_SOURCE_HASH
#define MLORA_SOURCE_HASH "unknown"
#endif
extern "C" const char *mlora_source_hash(void) { return MLORA_SOURCE_HASH; }

extern "C" const char *mlora_status_string(int status) {
  switch (status) {
    case MLORA_OK: return "ok";
    case MLORA_ERR_INVALID: return "invalid argument (null pointer, shape, stride or routing)";
    case MLORA_ERR_UNSUPPORTED: return "unsupported dtype or alignment";
    case MLORA_ERR_WORKSPACE: return "workspace missing or too small";
    case MLORA_ERR_LAUNCH: return "kernel launch failed";
    case MLORA_ERR_LIMIT: return "segment/adapter/rank limit of one call exceeded";
    case MLORA_ERR_DEVICE: return "no current device, or the device set-up of the library failed";
    default: return "unknown status";
  }
}
