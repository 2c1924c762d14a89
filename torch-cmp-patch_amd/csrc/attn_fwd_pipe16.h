// Software-pipelined fused attention forward for fp16 / bf16 on gfx950
// (v_mfma_f32_32x32x16_{f16,bf16}).
//
// Same register layout as attn_fwd_mfma16.h (S^T = K Q^T so that a lane owns
// one query row, O^T = V^T P^T, bit-permuted K feed, V^T fragments through
// ds_read_b64_tr_b16, optional Q pre-scaling with -m carried in the
// accumulator).  One wave owns 32 query rows; a workgroup of NW waves owns
// NW * 32.
//
// Schedule.  K runs one tile ahead of V, and a tile's exponentials are split
// over two iterations:
//
//   iteration t:  barrier
//                 read K(t+1) fragments; store K(t+2), V(t+1) to LDS;
//                 issue global loads of K(t+4), V(t+3)
//                 [ QK(t+1) MFMAs | exp/pack/row-sum, late half of tile t  ]
//                 check tile t (below)
//                 [ PV(t) MFMAs   | exp/pack/row-sum, early half of t+1   ]
//
// so that every MFMA has independent VALU work beside it in the same wave.
// Each bracketed part is issued in a fixed order (sched_barrier fences
// between MFMA-sized steps).  LDS holds two K and two V tiles; K(t+2) goes
// into the buffer K(t) left, V(t+1) into the one V(t-1) left, and the single
// barrier per iteration orders those writes after the previous iteration's
// reads.  With OPT bit 8 (below) the tiles instead load from memory straight
// into a four-tile LDS ring with a barrier every second iteration: even
// iterations issue K(t+3), K(t+4), V(t+2), V(t+3) and nothing is stored.
//
// Softmax without a per-tile max.  Tile 0 sets the row offset m from its max;
// later tiles are exponentiated as exp2(s*c - m) straight away.  The row sum
// of a lane's probabilities bounds every one of them, so a sum at most 2^8
// proves they all are, exactly what the max-first rule (rescale when the tile
// max exceeds m by more than 8 log2 units) would have accepted without a
// rescale.  A larger sum (rare) sends the wave to the exact path: tile max,
// rescale of O and l if it exceeds m + 8, tile redone.  Every rescale
// decision equals the max-first scheme's; the per-score max and the
// cross-lane reduction leave the common path.
//
// Key split.  When the query blocks do not fill whole rounds of the chip
// (e.g. 640 blocks on 256 CUs x 3 slots: 128 CUs would run 3 and 128 run 2),
// the blocks past the last whole round are cut into key ranges run by
// separate workgroups, so that every CU ends with the same work.  Each part
// leaves (O, m, l) in a workspace; the last part of a block to finish merges
// (per-wave counter, no waiting) and writes the output.
//
// Reference algorithm: src/cuda/fp16_flash_attention_hfma2.cu:72-243.
#pragma once

#include <type_traits>

#include "attn_fwd_mfma16.h"

namespace cmpext3 {

// OPT bit 0: s_setprio(1) around the MFMA-heavy block.  OPT bit 1: unpadded
// XOR-swizzled LDS rows (DK == DP in {32, 64, 128}).  OPT bit 2: leave the
// interleave to the compiler (no sched_barrier fences).  OPT bit 3: the head
// dim is not a multiple of 16 (D < DK), so K columns past D are zeroed.
// OPT bit 4: an attention mask (p.mask) is applied to every tile's scores
// before the exponentials (with CAUSAL, a pair must pass both).  OPT bit 5: each row's
// log-sum-exp goes to p.lse (the training forward).  OPT bit 6: narrow rows
// (FwdParams::elem_rows 4 or 8: head dims that are not whole 16-byte chunks,
// rows or base pointers off 16 bytes): K/V tiles are read as 4-byte pieces,
// K pieces past the head dim at an out-of-range offset (so they read as zero
// with no per-tile work), Q and O through ld_cols16 / st_cols16x4.  OPT bit
// 7: a single short query block (decode, packed query groups; the host sends
// it with at least two of the NW waves holding no rows): those rowless waves
// are the only ones that load and store K/V tiles, LDEPTH tiles ahead in
// registers the waves with rows need for their scores, and the waves with
// rows only compute.  OPT bit 8: K/V tiles go from memory straight into LDS
// (buffer_load_dwordx4 ... lds: lane i of an instruction writes the 16 bytes
// at M0 + 16 i) into a ring of four K and four V tiles, two tiles per
// barrier, with no staging registers and no LDS store instructions; every
// wave issues the same number of these loads per tile and waits for its own
// with an explicit vmcnt before the barrier that publishes them (the
// compiler does not track LDS written this way).  OPT bit 10 (with bits 4
// and 8): the mask is the same for every query row (m_q = 0, or one row)
// and read in whole runs: wave 0 loads each tile's slice of the mask row
// into a ring beside K, and the waves read it from LDS after the barrier.
// One workgroup's work on one query block: key tiles [g.tbase, g.tbase +
// g.ntiles) of block (g.bh, g.qblk).  With g.nparts > 1 that is key range
// g.part of the block's g.nparts, exchanged through row g.sb of the exchange
// space (g.pstride part slots per row).
struct Pipe16Seg {
  int bh, qblk, part, nparts, pstride, sb, tbase, ntiles;
};

template <typename T, int DK, int DP, int NW, int BK, int OCC, bool CAUSAL, bool PRESCALE, int OPT = 0>
__device__ __forceinline__ void pipe16_segment(const FwdParams& p, const SplitArgs& sa, const Pipe16Seg& g) {
  constexpr int NT = NW * 64;
  constexpr int BQ = NW * 32;
  constexpr bool SWZ = (OPT & 2) && (DK == DP) && (DK == 32 || DK == 64 || DK == 128);
  constexpr bool MASK = (OPT & 16) != 0;
  constexpr bool NARROW = (OPT & 64) != 0;
  // K/V tile row strides (halves): rows padded by 16 bytes, by 48 at D = 128
  // (fewer LDS bank conflicts there: 2-3% faster on causal bf16 D = 128,
  // no change at D = 64)
  constexpr int PAD = DK == 128 ? 24 : 8;
  constexpr int RSK = SWZ ? DK : DK + PAD;
  constexpr int RSV = SWZ ? DP : DP + PAD;
  constexpr int KTILE = BK * RSK;
  constexpr int VTILE = BK * RSV;
  constexpr int KCH = DK / 8;             // 16-byte chunks per K row
  constexpr int VCH = DP / 8;
  constexpr int KLD = (BK * KCH + NT - 1) / NT;
  constexpr int VLD = (BK * VCH + NT - 1) / NT;
  constexpr bool KFULL = BK * KCH % NT == 0;
  constexpr bool VFULL = BK * VCH % NT == 0;
  constexpr int NKB = BK / 32;            // 32-key blocks per tile
  constexpr int NCH = BK / 16;            // 16-key PV slices per tile
  constexpr int NDB = DP / 32;            // 32-row output blocks
  constexpr int NKS = DK / 16;            // score k-steps
  static_assert(BK % 32 == 0 && DK % 16 == 0 && DP % 32 == 0 && DK <= DP, "tile shape");
  constexpr bool DMA = (OPT & 256) != 0;
  static_assert(!(DMA && (NARROW || (OPT & 128))), "LDS DMA: whole-chunk rows, every wave computing");
  constexpr bool STREAMK = (OPT & 512) != 0;  // segments of an equal-work split (kernel below)
  constexpr int NR = DMA ? 4 : 2;  // K (and V) tiles held in LDS
  // With DMA: one barrier per two tiles.  The barrier before an even
  // iteration t publishes K(t+1), K(t+2), V(t), V(t+1) at once; right after
  // it the loads of K(t+3), K(t+4), V(t+2), V(t+3) go into the four slots
  // the two previous iterations finished reading, and each wave waits for all
  // of its loads before the next barrier, two iterations later (measured
  // 2-4% faster than a barrier per tile with loads three tiles ahead)

  // masked DMA launches: a ring of NR 128-byte slices of the mask, one per
  // tile (query-broadcast masks; see add_mask)
  constexpr int MSLOT = (MASK && DMA) ? 64 : 0;  // halves per mask slice
  __shared__ __attribute__((aligned(16))) uint16_t lds[NR * KTILE + NR * VTILE + NR * MSLOT];
  uint16_t* const kbase = lds;                // K(j) at kbase + (j % NR) * KTILE
  uint16_t* const vbase = lds + NR * KTILE;   // V(j) at vbase + (j % NR) * VTILE
  uint16_t* const mbase = lds + NR * (KTILE + VTILE);  // mask slice of tile j at mbase + (j % NR) * MSLOT

  const int tid = thread_x();
  const int wave = tid >> 6;
  const int lane = tid & 63;
  const int l32 = lane & 31;
  const int hh = lane >> 5;

  const int bh = g.bh, qblk = g.qblk, part = g.part, nparts = g.nparts;
  const int b = bh / p.H;
  const int h = bh - b * p.H;
  const int q0 = qblk * BQ;

  const uint16_t* __restrict__ qg = (const uint16_t*)p.q + b * p.q_b + h * p.q_h;
  const uint16_t* kg = (const uint16_t*)p.k + b * p.k_b + (h / p.kv_group) * p.k_h;
  const uint16_t* vg = (const uint16_t*)p.v + b * p.v_b + (h / p.kv_group) * p.v_h;
  uint16_t* __restrict__ og = (uint16_t*)p.o + b * p.o_b + h * p.o_h;

  const int Sq = p.Sq, Sk = p.Sk, D = p.D;
  const int qlo = q0 + wave * 32;          // first query row of this wave
  const int qrow = qlo + l32;
  const bool live = !(OPT & 128) || qlo < Sq;  // wave-uniform
  // element offset of row r: packed grouped-query rows interleave the group's
  // query heads (query head r / pack_sq, position r % pack_sq)
  auto row_off = [&](int r, int64_t s_head, int64_t s_row) -> int64_t {
    if (p.pack_sq > 0) {
      const int g = r / p.pack_sq;
      return g * s_head + (int64_t)(r - g * p.pack_sq) * s_row;
    }
    return (int64_t)r * s_row;
  };

  int kend = Sk;
  if (CAUSAL) kend = min(Sk, q0 + BQ);
  const int tbase = g.tbase, ntiles = g.ntiles;
  if (ntiles <= 0) return;  // Sk == 0 is rejected by the host
  // end of this workgroup's key range: the padding tile past it is masked
  const int kpe = min(kend, (tbase + ntiles) * BK);
  const int nt2 = (ntiles + 1) & ~1;  // iterations run (even)

  // ---- Q as the B operand of S^T = K Q^T
  const float cq = p.q_sign ? -p.c : p.c;
  u32x4 qf[NKS];
#pragma unroll
  for (int s = 0; s < NKS; ++s) {
    const int d = 16 * s + 8 * hh;
    u32x4 x = {0u, 0u, 0u, 0u};
    if (qrow < Sq && d < D) {
      const uint16_t* src = qg + row_off(qrow, p.q_g, p.q_s) + d;
      x = NARROW ? ld_cols16(src, D - d, p.elem_rows) : *(const u32x4*)src;
    }
    if (PRESCALE) {
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        const f32x2 f = Elt<T>::unpack(x[w]) * cq;
        x[w] = Elt<T>::pack(f[0], f[1]);
      }
    } else {
      x ^= p.q_sign;
    }
    qf[s] = x;
  }

  f32x16 oacc[NDB];
#pragma unroll
  for (int db = 0; db < NDB; ++db) oacc[db] = (f32x16){};
  f32x16 bias = (f32x16){};
  float mb = 0.f;
  // row sum of P over this lane's half of the keys: each tile's two
  // interleaved v_dot2 chains (tc0, tc1) are added once, after the rescale
  // check that needs their sum anyway
  float ls = 0.f;
  // rescale threshold on the tile's row max over the offset: -inf until the
  // row has seen a live key (the first live tile sets the offset), then 8
  float thr = -INFINITY;
  const float c = p.c;

  // ---- K/V tiles are fetched with raw buffer loads over this head's rows:
  // rows at or past Sk lie outside the buffer range and read as zero, every
  // load is unconditional (so the compiler counts them exactly across the
  // prefetch distance), and the tile offset is a scalar.  The host keeps
  // (Sk + BK) * row stride * 2 below 2^31.
  const int ks_b = (int)p.k_s * 2, vs_b = (int)p.v_s * 2;  // row strides in bytes
  const __amdgpu_buffer_rsrc_t krs = uniform_rsrc(kg, ((int64_t)(Sk - 1) * p.k_s + D) * 2);
  const __amdgpu_buffer_rsrc_t vrs = uniform_rsrc(vg, ((int64_t)(Sk - 1) * p.v_s + D) * 2);
  int kvo[KLD], klo[KLD];
  bool kz[KLD];  // chunk lies in the zero-filled head-dim columns
  // NARROW: byte offset of each 4-byte K piece; a piece past the head dim
  // gets an offset beyond every buffer range (the host keeps ranges below
  // 2^31, and 2^31 plus a tile offset stays below 2^32), so it reads zero
  int kvp[NARROW ? KLD : 1][4];
#pragma unroll
  for (int it = 0; it < KLD; ++it) {
    const int ci = it * NT + tid;
    const int r = ci / KCH, c8 = ci - r * KCH;
    kz[it] = 8 * c8 >= D;
    kvo[it] = r * ks_b + 16 * c8;
    klo[it] = r * RSK + 8 * (SWZ ? (c8 ^ lds_swz<DK>(r)) : c8);
    if constexpr (NARROW) {
#pragma unroll
      for (int w = 0; w < 4; ++w) kvp[it][w] = 8 * c8 + 2 * w < D ? kvo[it] + 4 * w : (int)0x80000000u;
    }
  }
  int vvo[VLD], vlo[VLD];
#pragma unroll
  for (int it = 0; it < VLD; ++it) {
    const int ci = it * NT + tid;
    const int r = ci / VCH, c8 = ci - r * VCH;
    vvo[it] = r * vs_b + 16 * c8;
    vlo[it] = r * RSV + 8 * (SWZ ? (c8 ^ lds_swz<DP>(r)) : c8);
  }
  // tile j (clamped to the last one) into a register set
  auto load_k = [&](int j, u32x4 (&kr)[KLD]) {
    const int so = (tbase + min(j, ntiles - 1)) * BK * ks_b;
#pragma unroll
    for (int it = 0; it < KLD; ++it) {
      if constexpr (NARROW) {
#pragma unroll
        for (int w = 0; w < 4; ++w) kr[it][w] = __builtin_amdgcn_raw_buffer_load_b32(krs, kvp[it][w], so, 0);
      } else {
        kr[it] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(krs, kvo[it], so, 0));
      }
    }
  };
  // NARROW: V pieces past the head dim read whatever follows (other rows, or
  // zero past the buffer range); they only feed output columns never stored
  auto load_v = [&](int j, u32x4 (&vr)[VLD]) {
    const int so = (tbase + min(j, ntiles - 1)) * BK * vs_b;
#pragma unroll
    for (int it = 0; it < VLD; ++it) {
      if constexpr (NARROW) {
#pragma unroll
        for (int w = 0; w < 4; ++w) vr[it][w] = __builtin_amdgcn_raw_buffer_load_b32(vrs, vvo[it] + 4 * w, so, 0);
      } else {
        vr[it] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(vrs, vvo[it], so, 0));
      }
    }
  };
  // K columns past D are zeroed (Q is zero there, and 0 * finite = 0 keeps
  // the padded k-steps exact); V columns past D only feed discarded outputs.
  auto store_k = [&](int slot, const u32x4 (&kr)[KLD]) {
    uint16_t* dst = kbase + slot * KTILE;
#pragma unroll
    for (int it = 0; it < KLD; ++it)
      if (KFULL || it * NT + tid < BK * KCH) {
        u32x4 x = kr[it];
        if ((OPT & 8) && kz[it]) x = (u32x4){0u, 0u, 0u, 0u};
        *(u32x4*)(dst + klo[it]) = x;
      }
  };
  auto store_v = [&](int j, const u32x4 (&vr)[VLD]) {
    uint16_t* dst = vbase + (j & 1) * VTILE;
#pragma unroll
    for (int it = 0; it < VLD; ++it)
      if (VFULL || it * NT + tid < BK * VCH) *(u32x4*)(dst + vlo[it]) = vr[it];
  };

  // OPT 256: a tile in LDS is BK rows of RSK (RSV) halves, i.e. NSK (NSV)
  // 16-byte slots counted row by row (padding included).  Wave w fills slots
  // [w * SPWK, (w + 1) * SPWK) with DIK instructions of 64 lanes (the last
  // one partial when SPWK is not a multiple of 64); since a tile has 32 rows,
  // every wave gets the same slot count.  Each lane's source chunk is fixed for the whole sweep (the tile
  // offset is the scalar soffset): padding slots, and K columns past D when
  // they must be zero, get an offset beyond every buffer range, which writes
  // zeros.
  constexpr int RCK = RSK / 8, RCV = RSV / 8;
  constexpr int NSK = BK * RCK, NSV = BK * RCV;
  constexpr int SPWK = NSK / NW, SPWV = NSV / NW;
  static_assert(!DMA || (NSK % NW == 0 && NSV % NW == 0 && RSK % 8 == 0 && RSV % 8 == 0), "DMA slot split");
  constexpr int DIK = DMA ? (SPWK + 63) / 64 : 1;
  constexpr int DIV = DMA ? (SPWV + 63) / 64 : 1;
  const int wv = __builtin_amdgcn_readfirstlane(wave);
  int dko[DIK], dvo[DIV];
  if constexpr (DMA) {
#pragma unroll
    for (int i = 0; i < DIK; ++i) {
      const int j = 64 * i + lane, sl = wv * SPWK + j;
      const int r = sl / RCK, cp = sl - r * RCK;
      const int c = SWZ ? (cp ^ lds_swz<DK>(r)) : cp;
      dko[i] = (j < SPWK && cp < KCH && !((OPT & 8) && 8 * c >= D)) ? r * ks_b + 16 * c : (int)0x80000000u;
    }
#pragma unroll
    for (int i = 0; i < DIV; ++i) {
      const int j = 64 * i + lane, sl = wv * SPWV + j;
      const int r = sl / RCV, cp = sl - r * RCV;
      const int c = SWZ ? (cp ^ lds_swz<DP>(r)) : cp;
      dvo[i] = (j < SPWV && cp < VCH) ? r * vs_b + 16 * c : (int)0x80000000u;
    }
  }
  typedef __attribute__((address_space(3))) uint16_t lds_u16;
  const uint32_t lds0 = (uint32_t)(uintptr_t)(lds_u16*)lds;  // LDS byte address of the tiles
  const u32x4 krw = uniform_rsrc_words(kg, ((int64_t)(Sk - 1) * p.k_s + D) * 2);
  const u32x4 vrw = uniform_rsrc_words(vg, ((int64_t)(Sk - 1) * p.v_s + D) * 2);
  // tile j (clamped to the last one) into ring slot `slot`
  auto dma_k = [&](int j, int slot) {
    const int so = (tbase + min(j, ntiles - 1)) * BK * ks_b;
#pragma unroll
    for (int i = 0; i < DIK; ++i)
      if (64 * i + lane < SPWK) lds_dma16(krw, lds0 + 2 * (slot * KTILE + (wv * SPWK + 64 * i) * 8), dko[i], so);
  };
  auto dma_v = [&](int j, int slot) {
    const int so = (tbase + min(j, ntiles - 1)) * BK * vs_b;
#pragma unroll
    for (int i = 0; i < DIV; ++i)
      if (64 * i + lane < SPWV)
        lds_dma16(vrw, lds0 + 2 * (NR * KTILE + slot * VTILE + (wv * SPWV + 64 * i) * 8), dvo[i], so);
  };
  // Query-broadcast masks (every row the same: m_q = 0, or one row) read in
  // whole runs: wave 0 brings tile j's BK keys of the mask row (BK * element
  // size bytes, at most 128) into ring slot `slot` with K(j), 4 bytes per
  // lane, so that the waves read them from LDS after the barrier that
  // publishes K(j) instead of waiting on a memory load inside the step.
  constexpr bool MBC = (OPT & 1024) != 0;  // the host sends only such masks with this bit
  static_assert(!MBC || (MASK && DMA), "mask slices ride the LDS DMA ring");
  const bool mbc = MBC;
  const int mbytes = p.mask_kind == MASK_BOOL ? 1 : p.mask_kind == MASK_F32 ? 4 : 2;
  const u32x4 mrw = uniform_rsrc_words(MASK ? (const void*)((const char*)p.mask + (b * p.m_b + h * p.m_h) * mbytes)
                                            : (const void*)p.q,
                                       MASK ? mask_span(p, mbytes) : 0);
  auto dma_m = [&](int j, int slot) {
    if (mbc && wv == 0 && lane < BK * mbytes / 4) {
      int vo = 4 * lane;
      asm volatile("" : "+v"(vo));  // computed here, not held through the loop
      lds_dma4(mrw, lds0 + 2 * (NR * (KTILE + VTILE) + slot * MSLOT), vo, (tbase + min(j, ntiles - 1)) * BK * mbytes);
    }
  };

  // OPT 128: the rowless waves (ltid = their thread index, nlt = their
  // thread count, at least 128) move every chunk of a tile.  Chunks past the
  // tile get an offset beyond every buffer range: they read zero, fetch
  // nothing and are not stored.
  constexpr bool LOADERS = (OPT & 128) != 0;
  static_assert(!(LOADERS && (NARROW || MASK || CAUSAL)), "loader waves: plain non-causal launches only");
  // tiles in flight per loader wave (its register ring): 4 at D <= 64, where
  // a tile is small (decode fp16 D = 64: 50 -> 43 us against the compute
  // waves loading two tiles ahead), 2 above (at D = 128 a deeper ring was
  // slower: 32k-key decode 108 us at 2, 110 at 3, 112 at 4, 118 at 6)
  constexpr int LDEPTH = DK <= 64 ? 4 : 2;
  constexpr int LKLD = LOADERS ? (BK * KCH + 127) / 128 : 1;
  constexpr int LVLD = LOADERS ? (BK * VCH + 127) / 128 : 1;
  const int nlive = LOADERS ? min(NW, (Sq - q0 + 31) / 32) : NW;
  const int ltid = tid - nlive * 64, nlt = (NW - nlive) * 64;
  int lkvo[LKLD], lklo[LKLD], lvvo[LVLD], lvlo[LVLD];
  bool lkz[LKLD];
  if constexpr (LOADERS) {
#pragma unroll
    for (int it = 0; it < LKLD; ++it) {
      const int ci = it * nlt + ltid, r = ci / KCH, c8 = ci - r * KCH;
      lkz[it] = 8 * c8 >= D;
      lkvo[it] = ci < BK * KCH ? r * ks_b + 16 * c8 : (int)0x80000000u;
      lklo[it] = ci < BK * KCH ? r * RSK + 8 * (SWZ ? (c8 ^ lds_swz<DK>(r)) : c8) : -1;
    }
#pragma unroll
    for (int it = 0; it < LVLD; ++it) {
      const int ci = it * nlt + ltid, r = ci / VCH, c8 = ci - r * VCH;
      lvvo[it] = ci < BK * VCH ? r * vs_b + 16 * c8 : (int)0x80000000u;
      lvlo[it] = ci < BK * VCH ? r * RSV + 8 * (SWZ ? (c8 ^ lds_swz<DP>(r)) : c8) : -1;
    }
  }
  auto lload_k = [&](int j, u32x4 (&kr)[LKLD]) {
    const int so = (tbase + min(j, ntiles - 1)) * BK * ks_b;
#pragma unroll
    for (int it = 0; it < LKLD; ++it)
      kr[it] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(krs, lkvo[it], so, 0));
  };
  auto lload_v = [&](int j, u32x4 (&vr)[LVLD]) {
    const int so = (tbase + min(j, ntiles - 1)) * BK * vs_b;
#pragma unroll
    for (int it = 0; it < LVLD; ++it)
      vr[it] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(vrs, lvvo[it], so, 0));
  };
  auto lstore_k = [&](int slot, const u32x4 (&kr)[LKLD]) {
    uint16_t* dst = kbase + slot * KTILE;
#pragma unroll
    for (int it = 0; it < LKLD; ++it)
      if (lklo[it] >= 0) {
        u32x4 x = kr[it];
        if ((OPT & 8) && lkz[it]) x = (u32x4){0u, 0u, 0u, 0u};
        *(u32x4*)(dst + lklo[it]) = x;
      }
  };
  auto lstore_v = [&](int j, const u32x4 (&vr)[LVLD]) {
    uint16_t* dst = vbase + (j & 1) * VTILE;
#pragma unroll
    for (int it = 0; it < LVLD; ++it)
      if (lvlo[it] >= 0) *(u32x4*)(dst + lvlo[it]) = vr[it];
  };

  // lane-constant parts of the fragment read addresses
  int k_rd[NKS];
  {
    const int r = perm_row(l32);
#pragma unroll
    for (int s = 0; s < NKS; ++s)
      k_rd[s] = r * RSK + (SWZ ? 8 * ((2 * s + hh) ^ lds_swz<DK>(r)) : 16 * s + 8 * hh);
  }
  const int jj = lane & 15, gg = lane >> 4;
  int v_rd[NDB][2];
#pragma unroll
  for (int db = 0; db < NDB; ++db)
#pragma unroll
    for (int half = 0; half < 2; ++half) {
      const int r = 8 * (gg >> 1) + (jj >> 2) + 4 * half;
      const int col = 32 * db + 16 * (gg & 1) + 4 * (jj & 3);
      v_rd[db][half] = r * RSV + (SWZ ? 8 * ((col >> 3) ^ lds_swz<DP>(r)) + (col & 7) : col);
    }

  auto read_kf = [&](int slot, u32x4 (&kf)[NKB][NKS]) {
    const uint16_t* ks = kbase + slot * KTILE;
#pragma unroll
    for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
      for (int s = 0; s < NKS; ++s) kf[kb][s] = *(const u32x4*)(ks + 32 * kb * RSK + k_rd[s]);
  };
  auto qk = [&](const u32x4 (&kf)[NKB][NKS], f32x16 (&sc)[NKB]) {
#pragma unroll
    for (int kb = 0; kb < NKB; ++kb) {
      f32x16 acc = PRESCALE ? bias : (f32x16){};
#pragma unroll
      for (int s = 0; s < NKS; ++s) acc = Elt<T>::mma(kf[kb][s], qf[s], acc);
      sc[kb] = acc;
    }
  };
  // exp2-domain scores x = s*c - m (PRESCALE: the accumulator already is)
  auto to_exp2 = [&](f32x16 (&sc)[NKB]) {
    if (!PRESCALE) {
#pragma unroll
      for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
        for (int r = 0; r < 16; ++r) sc[kb][r] = __builtin_fmaf(sc[kb][r], c, -mb);
    }
  };
  auto tile_needs_mask = [&](int j) {
    const int k0 = (tbase + j) * BK;
    return (k0 + BK > kpe) || (CAUSAL && k0 + BK - 1 > qlo);
  };
  // The lane's key base is laundered through an empty asm inside the (rarely
  // taken) branch: written plainly, the compiler hoists the 16 per-element key
  // computations out of the branch and every tile pays for them.
  auto mask = [&](int j, f32x16 (&sc)[NKB]) {
    int k0 = (tbase + j) * BK + 8 * hh;
    asm volatile("" : "+v"(k0));
#pragma unroll
    for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int key = k0 + 32 * kb + acc_key(r, 0);
        if (key >= kpe || (CAUSAL && key > qrow)) sc[kb][r] = -INFINITY;
      }
  };
  // attention mask of tile j added to (bool: applied to) exp2-domain scores.
  // A lane's 16 keys per 32-key block are 2 runs of 8 consecutive keys
  // (acc_key: 16j + 8hh + 0..7), so each run is one 8/16/32-byte read (or
  // one read per element for a narrow mask: mask_run8); rows past Sq use the
  // last row (their output is never stored).  Reads past the mask's readable
  // span (mask_span) return zero, and every key at or past Sk is masked by
  // the key-range rule afterwards.
  const int mes = p.mask_kind == MASK_BOOL ? 1 : p.mask_kind == MASK_F32 ? 4 : 2;
  const __amdgpu_buffer_rsrc_t mrs =
      uniform_rsrc(MASK ? (const void*)((const char*)p.mask + (b * p.m_b + h * p.m_h) * mes) : p.q,
                   MASK ? mask_span(p, mes) : 0);
  const int mrow_off = MASK ? (int)((int64_t)min(qrow, Sq - 1) * p.m_q * mes) : 0;
  // Whole runs are loaded first and applied only when some lane's keys of
  // the tile are dropped or biased (a wave-uniform test): a key-padding mask
  // leaves every tile before its padding untouched, and those tiles skip the
  // 16 selects or FMAs per 32-key block.
  auto add_mask = [&](int j, f32x16 (&sc)[NKB]) {
    const int k0 = (tbase + j) * BK;
    if constexpr (MBC) {
      // the tile's slice of the (query-broadcast) mask row, from LDS: tested
      // first, read again only to apply (LDS reads are cheap; registers are not)
      int o8 = 8 * hh * mes;
      asm volatile("" : "+v"(o8));  // computed here, not held through the loop
      const char* ms = (const char*)(mbase + (j & (NR - 1)) * MSLOT) + o8;
      auto run_at = [&](int kb, int run) {
        const char* r8 = ms + (32 * kb + 16 * run) * mes;
        MaskRun8 m;
        m.w1 = (u32x4){0u, 0u, 0u, 0u};
        if (p.mask_kind == MASK_BOOL) {
          const u32x2 w = *(const u32x2*)r8;
          m.w0 = (u32x4){w[0], w[1], 0x01010101u, 0x01010101u};
        } else {
          m.w0 = *(const u32x4*)r8;
          if (p.mask_kind == MASK_F32) m.w1 = *(const u32x4*)(r8 + 16);
        }
        return m;
      };
      bool keeps = true;
#pragma unroll
      for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
        for (int run = 0; run < 2; ++run) keeps = keeps && mask_run_keeps(run_at(kb, run), p.mask_kind);
      if (__builtin_amdgcn_ballot_w64(!keeps)) {
#pragma unroll
        for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
          for (int run = 0; run < 2; ++run) mask_apply8(sc[kb], 8 * run, run_at(kb, run), p.mask_kind);
      }
      return;
    }
    if constexpr (MBC) return;
    if (p.mask_narrow) {
#pragma unroll
      for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
        for (int run = 0; run < 2; ++run)  // keys k0 + 32 kb + 16 run + 8 hh .. + 7
          mask_run8(sc[kb], 8 * run, mrs, mrow_off + (k0 + 32 * kb + 16 * run + 8 * hh) * mes, p.mask_kind, true);
      return;
    }
    MaskRun8 mr[NKB][2];
    bool keeps = true;
#pragma unroll
    for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
      for (int run = 0; run < 2; ++run) {
        mr[kb][run] = mask_load8(mrs, mrow_off + (k0 + 32 * kb + 16 * run + 8 * hh) * mes, p.mask_kind);
        keeps = keeps && mask_run_keeps(mr[kb][run], p.mask_kind);
      }
    if (__builtin_amdgcn_ballot_w64(!keeps)) {
#pragma unroll
      for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
        for (int run = 0; run < 2; ++run) mask_apply8(sc[kb], 8 * run, mr[kb][run], p.mask_kind);
    }
  };
  // this lane's half of the row max (the two halves meet at the decision)
  auto row_max = [&](const f32x16 (&sc)[NKB]) {
    float m = -INFINITY;
#pragma unroll
    for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
      for (int r = 0; r < 16; ++r) m = fmaxf(m, sc[kb][r]);
    return m;
  };

  // ---- prologue: K(0), V(0), K(1) in LDS; register set A holds K(2), V(1)
  // for iteration 0 and set B holds K(3), V(2) for iteration 1
  u32x4 kA[KLD], vA[VLD], kB[KLD], vB[VLD];
  if constexpr (LOADERS) {
    if (!live) {
      // Loader waves: the same barrier sequence as the waves with rows (the
      // prologue's, then one per iteration), with ring set i % LDEPTH holding
      // K(i+2), V(i+1) for iteration i
      u32x4 lk[LDEPTH][LKLD], lv[LDEPTH][LVLD];
      lload_k(0, lk[0]);
      lload_v(0, lv[0]);
      lload_k(1, lk[1]);
      lstore_k(0, lk[0]);
      lstore_v(0, lv[0]);
      lstore_k(1, lk[1]);
#pragma unroll
      for (int j = 0; j < LDEPTH; ++j) {
        lload_k(j + 2, lk[j]);
        lload_v(j + 1, lv[j]);
      }
      lds_barrier();
      for (int t = 0; t < nt2; t += LDEPTH) {
#pragma unroll
        for (int j = 0; j < LDEPTH; ++j) {
          if (t + j < nt2) {
            lds_barrier();
            lstore_k((t + j) & 1, lk[j]);
            lstore_v(t + j + 1, lv[j]);
            lload_k(t + j + 2 + LDEPTH, lk[j]);
            lload_v(t + j + 1 + LDEPTH, lv[j]);
          }
        }
      }
      return;  // no rows: nothing to exchange or store
    }
  } else if constexpr (DMA) {
    // K(0) for the first scores, then what the barrier before iteration 0
    // publishes: K(1), K(2), V(0), V(1)
    dma_k(0, 0);
    dma_k(1, 1);
    dma_v(0, 0);
    dma_k(2, 2);
    dma_v(1, 1);
    dma_m(0, 0);
    dma_m(1, 1);
    dma_m(2, 2);
    wait_vmcnt<0>();
  } else {
    load_k(0, kA);
    load_v(0, vA);
    load_k(1, kB);
    store_k(0, kA);
    store_v(0, vA);
    store_k(1, kB);
    load_k(2, kA);
    load_v(1, vA);
    // set A must stay the older group: the loop waits for it with set B's loads
    // still counted as in flight
    __builtin_amdgcn_sched_barrier(0);
    load_k(3, kB);
    load_v(2, vB);
  }
  lds_barrier();
  constexpr int NQK = NKB * NKS;  // score MFMAs per tile
  constexpr int NPV = NCH * NDB;  // PV MFMAs per tile
  constexpr int NU = NCH * 4;     // exp units (2 exp + pack + row-sum step) per tile
  constexpr int NE = NU / 2;      // early units (first half of the chunks), done one iteration ahead
  static_assert(NCH % 2 == 0, "chunk split");

  // Raise the offset to the row max mx (never lower it once a live key was
  // seen) and rescale O and l; returns the shift applied to the scores.
  auto rescale = [&](float mx) {
    const bool fst = thr == -INFINITY;
    float delta = fst ? mx : fmaxf(mx, 0.f);
    if (mx == -INFINITY) delta = 0.f;
    const float alpha = fast_exp2(-delta);
    mb += delta;
    ls *= alpha;
#pragma unroll
    for (int db = 0; db < NDB; ++db) oacc[db] *= alpha;
    if (PRESCALE) bias -= delta;  // stays exactly -mb
    if (!(fst && mx == -INFINITY)) thr = 8.f;
    return delta;
  };
  // exp unit u of a tile: two probabilities, packed, into the tile's row sum
  auto unit = [&](int u, const f32x16 (&sc)[NKB], u32x4 (&pc)[NCH], float& t0, float& t1) {
    const int ch = u >> 2, e = u & 3, kb = ch >> 1, cc = ch & 1;
    const uint32_t w = Elt<T>::pack(fast_exp2(sc[kb][8 * cc + 2 * e]), fast_exp2(sc[kb][8 * cc + 2 * e + 1]));
    pc[ch][e] = w;
    if (e & 1) t1 = Elt<T>::sum2(w, t1);
    else t0 = Elt<T>::sum2(w, t0);
  };
  // bf16 path: the two scores of unit u into the exp2 domain
  auto conv = [&](int u, f32x16 (&sc)[NKB]) {
    if (!PRESCALE && !MASK) {
      const int ch = u >> 2, e = u & 3, kb = ch >> 1, cc = ch & 1;
      sc[kb][8 * cc + 2 * e] = __builtin_fmaf(sc[kb][8 * cc + 2 * e], c, -mb);
      sc[kb][8 * cc + 2 * e + 1] = __builtin_fmaf(sc[kb][8 * cc + 2 * e + 1], c, -mb);
    }
  };

  // tile 0 always sets the offset from its max
  f32x16 sA[NKB], sB[NKB];
  u32x4 pA[NCH], pB[NCH];
  float tA0 = 0.f, tA1 = 0.f, tB0 = 0.f, tB1 = 0.f;
  {
    u32x4 kf0[NKB][NKS];
    read_kf(0, kf0);
    qk(kf0, sA);
  }
  to_exp2(sA);
  if (MASK) add_mask(0, sA);
  if (tile_needs_mask(0)) mask(0, sA);
  {
    const float mx = xhalf_max(row_max(sA));
    const float delta = rescale(mx);
#pragma unroll
    for (int kb = 0; kb < NKB; ++kb) sA[kb] -= delta;
  }
#pragma unroll
  for (int u = 0; u < NE; ++u) unit(u, sA, pA, tA0, tA1);

  // One iteration.  On entry sc holds tile t's exp2-domain scores, pc the
  // early half of its probabilities and tc0/tc1 their row sums.
  auto step = [&](int t, f32x16 (&sc)[NKB], f32x16 (&sn)[NKB], u32x4 (&pc)[NCH], u32x4 (&pn)[NCH],
                  float& tc0, float& tc1, float& tn0, float& tn1, u32x4 (&kr)[KLD], u32x4 (&vr)[VLD]) {
    // every wave is done reading K(t) and V(t-1); K(t+1), V(t) are visible
    // (OPT 256: at even t only, after this wave's loads of K(t+1), K(t+2),
    // V(t), V(t+1) are complete; odd iterations read what that barrier
    // published)
    if constexpr (DMA) {
      if ((t & 1) == 0) {
        wait_vmcnt<0>();
        lds_barrier();
      }
    } else {
      lds_barrier();
    }
    u32x4 kf[NKB][NKS];
    read_kf((t + 1) & (NR - 1), kf);  // stale data on the last tile; those scores are dropped
    if constexpr (DMA) {
      // K(t+3) and K(t+4) into the slots K(t-1) and K(t) left, V(t+2) and
      // V(t+3) into those of V(t-2) and V(t-1); past the last tile a clamped
      // copy lands in a slot no later iteration reads
      if ((t & 1) == 0) {
        dma_k(t + 3, (t + 3) & (NR - 1));
        dma_v(t + 2, (t + 2) & (NR - 1));
        dma_k(t + 4, (t + 4) & (NR - 1));
        dma_v(t + 3, (t + 3) & (NR - 1));
        dma_m(t + 3, (t + 3) & (NR - 1));  // with K: read in the step before K's
        dma_m(t + 4, (t + 4) & (NR - 1));
      }
    } else if constexpr (!LOADERS) {
      // this iteration's register set holds K(t+2), V(t+1) (loaded two
      // iterations ago) and is refilled with K(t+4), V(t+3).  Past the last
      // tile the set holds a clamped copy that lands in a buffer no later
      // iteration reads, so the stores need no condition.  (OPT 128: the
      // loader waves do this instead.)
      store_k(t & 1, kr);
      store_v(t + 1, vr);
      load_k(t + 4, kr);
      load_v(t + 3, vr);
    }

    u32x4 vfr[NPV];
    const uint16_t* vs = vbase + (t & (NR - 1)) * VTILE;
    auto read_vfr = [&](int i) {
      const int ch = i / NDB, db = i - ch * NDB;
      const uint16_t* vp = vs + 16 * ch * RSV;
      const uint2 lo = lds_tr16_b64(vp + v_rd[db][0]);
      const uint2 hi = lds_tr16_b64(vp + v_rd[db][1]);
      vfr[i] = (u32x4){lo.x, lo.y, hi.x, hi.y};
    };
    // ---- stage A: score MFMAs of tile t+1 beside the V fragment reads of
    // tile t and the late half of tile t's exp units
    if (OPT & 1) __builtin_amdgcn_s_setprio(1);
    f32x16 acc[NKB];
#pragma unroll
    for (int i = 0; i < NQK; ++i) {
      const int kb = i / NKS, s = i - kb * NKS;
#pragma unroll
      for (int v = i * NPV / NQK; v < (i + 1) * NPV / NQK; ++v) read_vfr(v);
      acc[kb] = Elt<T>::mma(kf[kb][s], qf[s], s == 0 ? (PRESCALE ? bias : (f32x16){}) : acc[kb]);
#pragma unroll
      for (int u = i * NE / NQK; u < (i + 1) * NE / NQK; ++u) unit(NE + u, sc, pc, tc0, tc1);
      if (!(OPT & 4)) __builtin_amdgcn_sched_barrier(0);
    }
    if (OPT & 1) __builtin_amdgcn_s_setprio(0);
#pragma unroll
    for (int kb = 0; kb < NKB; ++kb) sn[kb] = acc[kb];

    // ---- tile t is exponentiated against the running offset without its
    // own max.  A lane row sum above 2^8 (always true if some probability
    // exceeds 2^8) sends the wave to the exact path: the tile max decides a
    // rescale as in the max-first scheme, and the tile is redone.
    // Without an attention mask every row sees a key in the first tile of its
    // sweep (key 0 under causal; rows past Sq score 0), so that tile already
    // set the offset and thr is 8; only a mask can leave it at -inf.
    float tsum = tc0 + tc1;
    if (__builtin_amdgcn_ballot_w64((MASK && thr == -INFINITY) || tsum > 256.f)) {
      const float mx = xhalf_max(row_max(sc));
      if (__builtin_amdgcn_ballot_w64(mx > thr)) {
        const float delta = rescale(mx);
#pragma unroll
        for (int kb = 0; kb < NKB; ++kb) sc[kb] -= delta;
        if (PRESCALE) {
#pragma unroll
          for (int kb = 0; kb < NKB; ++kb) sn[kb] -= delta;  // scored with the old offset
        }
        tc0 = 0.f;
        tc1 = 0.f;
#pragma unroll
        for (int u = 0; u < NU; ++u) unit(u, sc, pc, tc0, tc1);
        tsum = tc0 + tc1;
      }
    }
    ls += tsum;
    if (MASK) {
      // the mask is added in the exp2 domain, so masked bf16 tiles are
      // converted here rather than unit by unit in stage B
      if (t + 1 < nt2) {
        to_exp2(sn);
        add_mask(t + 1, sn);
        if (tile_needs_mask(t + 1)) mask(t + 1, sn);
      }
    } else if (t + 1 < nt2 && tile_needs_mask(t + 1)) {
      mask(t + 1, sn);
    }

    // ---- stage B: PV MFMAs of tile t beside the K(t+2) fragment reads and
    // the early half of tile t+1's exp units
    if (OPT & 1) __builtin_amdgcn_s_setprio(1);
    tn0 = 0.f;
    tn1 = 0.f;
#pragma unroll
    for (int i = 0; i < NPV; ++i) {
      const int ch = i / NDB, db = i - ch * NDB;
      oacc[db] = Elt<T>::mma(vfr[i], pc[ch], oacc[db]);
#pragma unroll
      for (int u = i * NE / NPV; u < (i + 1) * NE / NPV; ++u) {
        conv(u, sn);
        unit(u, sn, pn, tn0, tn1);
      }
      if (!(OPT & 4)) __builtin_amdgcn_sched_barrier(0);
    }
#pragma unroll
    for (int u = NE; u < NU; ++u) conv(u, sn);
    if (OPT & 1) __builtin_amdgcn_s_setprio(0);
  };

  // An even number of iterations keeps the loop body free of a mid-loop
  // exit, which would make the compiler wait for every prefetch at the top.
  // With an odd tile count the extra tile is a clamped copy of the last one
  // whose keys all lie past kpe: fully masked, it adds exactly zero.  The
  // last iteration's early units work on stale scores nobody reads.
  if constexpr (DMA) {
    // unrolled by the ring size so that every slot index is a constant; an
    // exit after an even number of iterations waits for nothing (the loads
    // write no registers)
    for (int t = 0; t < nt2; t += 4) {
      step(t, sA, sB, pA, pB, tA0, tA1, tB0, tB1, kA, vA);
      step(t + 1, sB, sA, pB, pA, tB0, tB1, tA0, tA1, kB, vB);
      if (t + 2 >= nt2) break;
      step(t + 2, sA, sB, pA, pB, tA0, tA1, tB0, tB1, kA, vA);
      step(t + 3, sB, sA, pB, pA, tB0, tB1, tA0, tA1, kB, vB);
    }
    // the clamped loads past the last tile are still writing this
    // workgroup's LDS: they must land before the wave can leave
    wait_vmcnt<0>();
  } else {
    for (int t = 0; t < nt2; t += 2) {
      step(t, sA, sB, pA, pB, tA0, tA1, tB0, tB1, kA, vA);
      step(t + 1, sB, sA, pB, pA, tB0, tB1, tA0, tA1, kB, vB);
    }
  }

  // ---- epilogue
  float lsum = xhalf_sum(ls);
  float moff = mb;  // exp2-domain offset of lsum
  // a wave whose rows all lie past Sq (short or packed query sweeps) has
  // nothing to exchange or store; every part of the block agrees on that
  if (qlo >= Sq) return;
  if (nparts > 1) {
    // Leave this part's state, then let the last part of the block merge
    // (its own state straight from its registers); no part ever waits for
    // another workgroup.  Two parts (the tail of a whole-round grid, where
    // each part holds up to 36 KB per 128-row block): the parts count their
    // arrivals first, so usually only the first writes and the second merges
    // (both write only when the second arrives while the first is still
    // writing).  More parts (short-query grids, whose parts end together):
    // every part writes, then counts itself in, and the last one in merges.
    // Device-scope (sc1) stores and loads keep the exchange coherent across
    // the XCDs' L2s without cache-wide write-back or invalidation.
    constexpr int NV = split_vectors(DP);
    static_assert(NV == NDB * 4 + 1, "O fragments + (m, l)");
    const int sb = g.sb, ps = g.pstride;
    const int nwl = sa.nwl;  // waves past it hold no rows and left above
    const __amdgpu_buffer_rsrc_t wsr = uniform_rsrc(sa.ws, (int64_t)(sb + 1) * ps * nwl * NV * 64 * 16);
    auto voff = [&](int q, int k) { return ((((sb * ps + q) * nwl + wave) * NV + k) * 64 + lane) * 16; };
    // Every lane moves its vectors, also lanes of rows past Sq (a decode
    // step's wave holds one or two live rows): whole 1 KB runs per
    // instruction measured faster than the sparse 16-byte pieces of the live
    // rows alone (decode step 49.1 vs 51.1 us), partial lines being costlier
    // to write through to memory than full ones.
    // device-scope (aux 16 = sc1) 16-byte accesses; the builtins move dwords, so the
    // fp32 values go through explicit bit casts
    auto st_ws = [&](f32x4 x, int off) {
      __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, x), wsr, off, 0, 16);
    };
    auto ld_ws = [&](int off) { return __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(wsr, off, 0, 16)); };
    int* const ctr = sa.cnt + 2 * (sb * nwl + wave);  // {parts arrived, states written}
    // a part whose keys are all masked for this row holds nothing: offset -inf
    const float m_own = lsum > 0.f ? mb : -INFINITY;
    // Two fp16 parts exchange their O normalised by their own row sum, in
    // fp16 (a quarter of the bytes): 2 * NDB vectors, then (m, l) as 8 bytes
    // per lane.  Both parts round their own O this way, so the result does
    // not depend on which one writes (reruns stay bit-identical); rounding O/l
    // to fp16 before the merge adds at most one fp16 rounding to the output.
    const bool half_x = std::is_same<T, _Float16>::value && (nparts == 2 || STREAMK);
    auto ml_off = [&](int q) {
      return ((((sb * ps + q) * nwl + wave) * NV + 2 * NDB) * 64) * 16 + lane * 8;
    };
    u32x4 own_h[2 * NDB];  // half_x: this part's O / l in fp16
    if (half_x) {
      const float il = lsum > 0.f ? 1.f / lsum : 0.f;
#pragma unroll
      for (int db = 0; db < NDB; ++db)
#pragma unroll
        for (int w = 0; w < 8; ++w)
          own_h[2 * db + w / 4][w % 4] = Elt<T>::pack(oacc[db][2 * w] * il, oacc[db][2 * w + 1] * il);
    }
    auto leave_state = [&]() {
      if (half_x) {
#pragma unroll
        for (int v = 0; v < 2 * NDB; ++v)
          __builtin_amdgcn_raw_buffer_store_b128(own_h[v], wsr, voff(part, v), 0, 16);
        __builtin_amdgcn_raw_buffer_store_b64((u32x2){__float_as_uint(m_own), __float_as_uint(lsum)}, wsr,
                                              ml_off(part), 0, 16);
      } else {
#pragma unroll
        for (int db = 0; db < NDB; ++db)
#pragma unroll
          for (int g = 0; g < 4; ++g)
            st_ws((f32x4){oacc[db][4 * g], oacc[db][4 * g + 1], oacc[db][4 * g + 2], oacc[db][4 * g + 3]},
                  voff(part, db * 4 + g));
        st_ws((f32x4){m_own, lsum, 0.f, 0.f}, voff(part, NDB * 4));
      }
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    };
    if (nparts == 2) {
      // Arrival order decides who writes; nobody waits.  The first to arrive
      // always leaves its state.  The second leaves it only if the first has
      // not finished writing yet (the written counter still 0).  Whoever
      // then completes the pair (finds the other's state written) merges.
      auto add = [&](int* c) {
        int old = 0;
        if (lane == 0) old = __hip_atomic_fetch_add(c, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        return __builtin_amdgcn_readfirstlane(old);
      };
      if (add(ctr) == 0) {
        leave_state();
        if (add(ctr + 1) == 0) return;  // the second part merges
      } else {
        int w = 0;
        if (lane == 0) w = __hip_atomic_load(ctr + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (__builtin_amdgcn_readfirstlane(w) == 0) {
          leave_state();
          if (add(ctr + 1) == 0) return;  // the first part merges
        }
      }
      if (lane == 0) {
        __hip_atomic_store(ctr, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store(ctr + 1, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
    } else {
      leave_state();
      int old = 0;
      if (lane == 0) old = __hip_atomic_fetch_add(ctr, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      old = __builtin_amdgcn_readfirstlane(old);
      if (old != nparts - 1) return;
      if (lane == 0) __hip_atomic_store(ctr, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    asm volatile("" ::: "memory");  // the exchange loads stay after the counters
    // Merge every part in part order, this one from its registers: the same
    // instructions on the same values whichever part arrives last, so a
    // rerun is bit-identical.
    auto ml_of = [&](int q) -> f32x2 {
      if (q == part) return (f32x2){m_own, lsum};
      if (half_x) {
        const u32x2 w = __builtin_bit_cast(u32x2, __builtin_amdgcn_raw_buffer_load_b64(wsr, ml_off(q), 0, 16));
        return (f32x2){__uint_as_float(w[0]), __uint_as_float(w[1])};
      }
      const f32x4 x = ld_ws(voff(q, NDB * 4));
      return (f32x2){x[0], x[1]};
    };
    // fp32 exchange: the loads of CH parts are issued together (one memory
    // round trip per CH parts, not per part); part indices past the last are
    // clamped to it and dropped, the own part's loads (of whatever its slot
    // holds) are replaced by its registers.
    constexpr int CH = 4;                   // parts per batch of offset loads
    constexpr int CH2 = NDB <= 2 ? 2 : 1;   // parts per batch of O loads (registers)
    float mt = m_own;
    if (half_x) {
      for (int q = 0; q < nparts; ++q)
        if (q != part) mt = fmaxf(mt, ml_of(q)[0]);
    } else {
      for (int q0 = 0; q0 < nparts; q0 += CH) {
        float mq[CH];
#pragma unroll
        for (int j = 0; j < CH; ++j) mq[j] = ld_ws(voff(min(q0 + j, nparts - 1), NDB * 4))[0];
#pragma unroll
        for (int j = 0; j < CH; ++j)
          if (q0 + j < nparts && q0 + j != part) mt = fmaxf(mt, mq[j]);
      }
    }
    moff = mt;
    f32x16 own[NDB];
#pragma unroll
    for (int db = 0; db < NDB; ++db) {
      own[db] = oacc[db];
      oacc[db] = (f32x16){};
    }
    float lnew = 0.f;
    if (half_x) {
      for (int q = 0; q < nparts; ++q) {  // O / l in fp16, weighted by a * l
        const f32x2 ml = ml_of(q);
        const float a = ml[0] == -INFINITY ? 0.f : fast_exp2(ml[0] - mt);
        lnew = __builtin_fmaf(ml[1], a, lnew);
        const float wq = a * ml[1];
#pragma unroll
        for (int v = 0; v < 2 * NDB; ++v) {
          const u32x4 x = q == part ? own_h[v]
                                    : __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(wsr, voff(q, v), 0, 16));
#pragma unroll
          for (int w = 0; w < 4; ++w) {
            const f32x2 f = Elt<T>::unpack(x[w]);
            const int i = 8 * (v & 1) + 2 * w;
            oacc[v / 2][i] = __builtin_fmaf(f[0], wq, oacc[v / 2][i]);
            oacc[v / 2][i + 1] = __builtin_fmaf(f[1], wq, oacc[v / 2][i + 1]);
          }
        }
      }
    } else {
      for (int q0 = 0; q0 < nparts; q0 += CH2) {
        f32x4 ml[CH2], x[CH2][NDB * 4];
#pragma unroll
        for (int j = 0; j < CH2; ++j) {
          const int qq = min(q0 + j, nparts - 1);
          ml[j] = ld_ws(voff(qq, NDB * 4));
#pragma unroll
          for (int v = 0; v < NDB * 4; ++v) x[j][v] = ld_ws(voff(qq, v));
        }
#pragma unroll
        for (int j = 0; j < CH2; ++j) {
          const int q = q0 + j;
          if (q >= nparts) break;
          const bool mine = q == part;
          const float mq = mine ? m_own : ml[j][0];
          const float a = mq == -INFINITY ? 0.f : fast_exp2(mq - mt);
          lnew = __builtin_fmaf(mine ? lsum : ml[j][1], a, lnew);
#pragma unroll
          for (int db = 0; db < NDB; ++db)
#pragma unroll
            for (int g = 0; g < 4; ++g)
#pragma unroll
              for (int i = 0; i < 4; ++i)
                oacc[db][4 * g + i] =
                    __builtin_fmaf(mine ? own[db][4 * g + i] : x[j][db * 4 + g][i], a, oacc[db][4 * g + i]);
        }
      }
    }
    lsum = lnew;
  }
  // a row that saw no key at all (every key masked) gives zeros, as torch does
  const float inv = lsum > 0.f ? 1.f / lsum : 0.f;
  // log-sum-exp in natural log: (offset + log2 of the sum) * ln 2
  if constexpr ((OPT & 32) != 0) {
    if (qrow < Sq && hh == 0)
      p.lse[(int64_t)bh * Sq + qrow] =
          lsum > 0.f ? (moff + __builtin_amdgcn_logf(lsum)) * 0.6931471805599453f : -INFINITY;
  }
  if (qrow < Sq) {
    uint16_t* orow = og + row_off(qrow, p.o_g, p.o_s);
#pragma unroll
    for (int db = 0; db < NDB; ++db)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int d = 32 * db + 8 * g + 4 * hh;
        if (d < D) {
          u32x2 w;
          w[0] = Elt<T>::pack(oacc[db][4 * g + 0] * inv, oacc[db][4 * g + 1] * inv);
          w[1] = Elt<T>::pack(oacc[db][4 * g + 2] * inv, oacc[db][4 * g + 3] * inv);
          if (NARROW)
            st_cols16x4(orow + d, w, D - d, p.elem_rows);
          else
            *(u32x2*)(orow + d) = w;
        }
      }
  }
}

// The kernel.  Without OPT bit 512 a workgroup owns one block, or one key
// range of a block past the whole rounds (SplitArgs::nfull / nparts).  With
// OPT bit 512 (stream-K, non-causal): the launch is a whole number of rounds
// of workgroups, and workgroup w takes the w-th of SplitArgs::sk_wgs equal
// shares of the sequence of (block, key tile) pairs, blocks in order, so
// every workgroup does the same number of tiles and the chip's slots all end
// together.  A share runs as segments, one per block it touches (at most two
// when a share is shorter than a block); a block cut between workgroups
// merges its parts as any key split does, in part order (part i of a block
// is the i-th workgroup that touches it), through row `block` of the
// exchange with SplitArgs::nparts part slots per row.
template <typename T, int DK, int DP, int NW, int BK, int OCC, bool CAUSAL, bool PRESCALE, int OPT = 0>
__global__ void __launch_bounds__(NW * 64) __attribute__((amdgpu_waves_per_eu(OCC)))
attn_fwd_pipe16(const FwdParams p, const SplitArgs sa) {
  if constexpr ((OPT & 512) != 0) {
    static_assert(!CAUSAL, "stream-K: non-causal launches only");
    const int W = sa.sk_wgs;
    const int ntall = (p.Sk + BK - 1) / BK;
    const int64_t tot = (int64_t)p.n_wg * ntall;  // block-tile pairs
    // adjacent shares on one XCD (workgroup i runs on XCD i % 8), so the
    // blocks of a head stream their K/V through one L2
    const int w = xcd_remap(block_x(), W);
    const int64_t end = (int64_t)(w + 1) * tot / W;
    // the first workgroup whose share holds tile position x
    auto owner = [&](int64_t x) { return (int)(((x + 1) * W - 1) / tot); };
    // the segment of this share that starts at tile position pos
    auto segment = [&](int64_t pos) {
      const int blk = (int)(pos / ntall);
      const int64_t x0 = (int64_t)blk * ntall;
      const int t1 = (int)(end - x0 < ntall ? end - x0 : ntall);
      const int wf = owner(x0);
      const Pipe16Seg g = {blk / p.n_qblk, blk % p.n_qblk, w - wf, owner(x0 + ntall - 1) - wf + 1,
                           sa.nparts, blk, (int)(pos - x0), t1 - (int)(pos - x0)};
      pipe16_segment<T, DK, DP, NW, BK, OCC, CAUSAL, PRESCALE, OPT>(p, sa, g);
      return x0 + t1;
    };
    // a share is at most one block long (the host plans it so), so it
    // touches at most two blocks
    const int64_t next = segment((int64_t)w * tot / W);
    if (next < end) {
      lds_barrier();  // every wave is done with the first segment's LDS
      segment(next);
    }
  } else {
    int lb = block_x(), part = 0, nparts = 1;
    if (lb >= sa.nfull) {
      const int r = lb - sa.nfull;
      nparts = sa.nparts;
      lb = sa.nfull + r / nparts;
      part = r - (lb - sa.nfull) * nparts;
    }
    int bh, qblk;
    wg_tile(lb, p, CAUSAL, bh, qblk);
    int kend = p.Sk;
    if (CAUSAL) kend = min(p.Sk, (qblk + 1) * NW * 32);
    const int ntall = (kend + BK - 1) / BK;
    const int tbase = part * ntall / nparts;
    const Pipe16Seg g = {bh, qblk, part, nparts, nparts, lb - sa.nfull, tbase,
                         (part + 1) * ntall / nparts - tbase};
    pipe16_segment<T, DK, DP, NW, BK, OCC, CAUSAL, PRESCALE, OPT>(p, sa, g);
  }
}

template <typename T, int DK, int NW, int BK, int OCC, bool CAUSAL, bool PRESCALE, int OPT = 0>
hipError_t launch_pipe16_cfg(const FwdParams& p0, const SplitArgs& sa, hipStream_t stream) {
  constexpr int DP = (DK + 31) / 32 * 32;
  constexpr int BQ = NW * 32;
  FwdParams p = p0;
  p.n_qblk = (p.Sq + BQ - 1) / BQ;
  p.n_wg = p.B * p.H * p.n_qblk;
  if (p.n_wg == 0) return hipSuccess;
  // buffer offsets of the K/V tiles are 32-bit
  const int64_t rs = p.k_s > p.v_s ? p.k_s : p.v_s;
  if ((int64_t)(p.Sk + BK) * rs * 2 >= (int64_t(1) << 31)) return hipErrorInvalidValue;
  if (p.dry) return hipSuccess;
  const int nwg = (OPT & 512) ? sa.sk_wgs : sa.nfull + (p.n_wg - sa.nfull) * sa.nparts;
  hipLaunchKernelGGL((attn_fwd_pipe16<T, DK, DP, NW, BK, OCC, CAUSAL, PRESCALE, OPT>), dim3(nwg),
                     dim3(NW * 64), 0, stream, p, sa);
  return hipGetLastError();
}

}  // namespace cmpext3
