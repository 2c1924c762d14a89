// Software-pipelined fused attention forward for fp16 / bf16 on gfx950
// (v_mfma_f32_32x32x16_{f16,bf16}).
//
// Same math and register layout as attn_fwd_mfma16.h (S^T = K Q^T so that a
// lane owns one query row, O^T = V^T P^T, bit-permuted K feed, V^T fragments
// through ds_read_b64_tr_b16, optional Q pre-scaling with -m carried in the
// accumulator, max-first lazy rescale).  One wave owns 32 query rows; a
// workgroup of NW waves owns NW * 32.
//
// The difference is the schedule.  In attn_fwd_mfma16 a wave's tile is a
// dependency chain (scores -> max -> exp -> PV), so the MFMA pipe and the VALU
// only overlap across waves.  Here K runs one tile ahead of V:
//
//   iteration t:  barrier
//                 read K(t+1) fragments; store K(t+2), V(t+1) to LDS;
//                 issue global loads of K(t+4), V(t+3)
//                 rescale decision for tile t (max computed last iteration)
//                 [ QK(t+1) MFMAs | exp/pack/row-sum of tile t ]
//                 [ PV(t) MFMAs   | row max of tile t+1        ]
//
// so that every MFMA of the tile has independent VALU work next to it in the
// same wave.  The bracketed part is one basic block issued in a fixed order
// (sched_barrier fences between MFMA-sized steps).  LDS holds two K and two V tiles; K(t+2) goes into
// the buffer K(t) left, V(t+1) into the one V(t-1) left, and the single
// barrier per iteration orders those writes after the previous iteration's
// reads.
//
// Reference algorithm: src/cuda/fp16_flash_attention_hfma2.cu:72-243.
#pragma once

#include "attn_fwd_mfma16.h"

namespace cmpext3 {

// Raw buffer resource over [base, base + bytes) (gfx9 dword3: 32-bit raw
// reads).  The fields go through readfirstlane so that the compiler keeps the
// descriptor in SGPRs instead of wrapping every load in a waterfall loop.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t uniform_rsrc(const void* base, int64_t bytes) {
  const uint64_t a = (uint64_t)base;
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)a);
  const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(a >> 32));
  const int n = __builtin_amdgcn_readfirstlane((int)bytes);
  return __builtin_amdgcn_make_buffer_rsrc((void*)(((uint64_t)hi << 32) | lo), (short)0, n, 0x00020000);
}

// OPT bit 0: s_setprio(1) around the MFMA-heavy block.  OPT bit 1: unpadded
// XOR-swizzled LDS rows (DK == DP in {32, 64, 128}).  OPT bit 2: leave the
// interleave to the compiler (no sched_barrier fences).  OPT bit 3: the head
// dim is not a multiple of 16 (D < DK), so K columns past D are zeroed.
template <typename T, int DK, int DP, int NW, int BK, int OCC, bool CAUSAL, bool PRESCALE, int OPT = 0>
__global__ void __launch_bounds__(NW * 64) __attribute__((amdgpu_waves_per_eu(OCC)))
attn_fwd_pipe16(const FwdParams p) {
  constexpr int NT = NW * 64;
  constexpr int BQ = NW * 32;
  constexpr bool SWZ = (OPT & 2) && (DK == DP) && (DK == 32 || DK == 64 || DK == 128);
  constexpr int RSK = SWZ ? DK : DK + 8;  // K tile row stride (halves)
  constexpr int RSV = SWZ ? DP : DP + 8;  // V tile row stride (halves)
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

  __shared__ __attribute__((aligned(16))) uint16_t lds[2 * KTILE + 2 * VTILE];
  uint16_t* const kbase = lds;               // K(j) at kbase + (j & 1) * KTILE
  uint16_t* const vbase = lds + 2 * KTILE;   // V(j) at vbase + (j & 1) * VTILE

  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  const int lane = tid & 63;
  const int l32 = lane & 31;
  const int hh = lane >> 5;

  int bh, qblk;
  wg_tile(blockIdx.x, p, CAUSAL, bh, qblk);
  const int b = bh / p.H;
  const int h = bh - b * p.H;
  const int q0 = qblk * BQ;

  const uint16_t* __restrict__ qg = (const uint16_t*)p.q + b * p.q_b + h * p.q_h;
  const uint16_t* kg = (const uint16_t*)p.k + b * p.k_b + h * p.k_h;
  const uint16_t* vg = (const uint16_t*)p.v + b * p.v_b + h * p.v_h;
  uint16_t* __restrict__ og = (uint16_t*)p.o + b * p.o_b + h * p.o_h;

  const int Sq = p.Sq, Sk = p.Sk, D = p.D;
  const int qlo = q0 + wave * 32;          // first query row of this wave
  const int qrow = qlo + l32;

  int kend = Sk;
  if (CAUSAL) kend = min(Sk, q0 + BQ);
  const int ntiles = (kend + BK - 1) / BK;
  if (ntiles <= 0) return;  // Sk == 0 is rejected by the host
  const int nt2 = (ntiles + 1) & ~1;  // iterations run (even)

  // ---- Q as the B operand of S^T = K Q^T
  const float cq = p.q_sign ? -p.c : p.c;
  u32x4 qf[NKS];
#pragma unroll
  for (int s = 0; s < NKS; ++s) {
    const int d = 16 * s + 8 * hh;
    u32x4 x = {0u, 0u, 0u, 0u};
    if (qrow < Sq && d < D) x = *(const u32x4*)(qg + (int64_t)qrow * p.q_s + d);
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
  // row sum of P over this lane's half of the keys, as two interleaved v_dot2
  // chains carried across iterations (no per-iteration reduction to wait on)
  float ls0 = 0.f, ls1 = 0.f;
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
#pragma unroll
  for (int it = 0; it < KLD; ++it) {
    const int ci = it * NT + tid;
    const int r = ci / KCH, c8 = ci - r * KCH;
    kz[it] = 8 * c8 >= D;
    kvo[it] = r * ks_b + 16 * c8;
    klo[it] = r * RSK + 8 * (SWZ ? (c8 ^ lds_swz<DK>(r)) : c8);
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
    const int so = min(j, ntiles - 1) * BK * ks_b;
#pragma unroll
    for (int it = 0; it < KLD; ++it)
      kr[it] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(krs, kvo[it], so, 0));
  };
  auto load_v = [&](int j, u32x4 (&vr)[VLD]) {
    const int so = min(j, ntiles - 1) * BK * vs_b;
#pragma unroll
    for (int it = 0; it < VLD; ++it)
      vr[it] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(vrs, vvo[it], so, 0));
  };
  // K columns past D are zeroed (Q is zero there, and 0 * finite = 0 keeps
  // the padded k-steps exact); V columns past D only feed discarded outputs.
  auto store_k = [&](int j, const u32x4 (&kr)[KLD]) {
    uint16_t* dst = kbase + (j & 1) * KTILE;
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

  auto read_kf = [&](int j, u32x4 (&kf)[NKB][NKS]) {
    const uint16_t* ks = kbase + (j & 1) * KTILE;
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
    const int k0 = j * BK;
    return (k0 + BK > Sk) || (CAUSAL && k0 + BK - 1 > qlo);
  };
  auto mask = [&](int j, f32x16 (&sc)[NKB]) {
    const int k0 = j * BK;
#pragma unroll
    for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int key = k0 + 32 * kb + acc_key(r, hh);
        if (key >= Sk || (CAUSAL && key > qrow)) sc[kb][r] = -INFINITY;
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
  lds_barrier();
  f32x16 sA[NKB], sB[NKB];
  {
    u32x4 kf[NKB][NKS];
    read_kf(0, kf);
    qk(kf, sA);
  }
  to_exp2(sA);
  if (tile_needs_mask(0)) mask(0, sA);
  float mq = row_max(sA);

  constexpr int NQK = NKB * NKS;  // score MFMAs per tile
  constexpr int NPV = NCH * NDB;  // PV MFMAs per tile
  constexpr int NU = NCH * 4;     // exp units (2 exp + pack + row-sum step) per tile
  // Units placed beside the score MFMAs; the rest go beside the PV MFMAs,
  // unit UA + i after PV MFMA i.  Unit u feeds 16-key chunk u / 4, whose
  // first PV MFMA has index NDB * (u / 4), so the last unit must land in an
  // earlier step.  With 3/4 of the units up front that holds when NDB >= 2;
  // with a single output block every unit goes up front.
  constexpr int UA = NDB > 1 ? (3 * NU) / 4 : NU;
  static_assert(NU - 1 - UA < (NU - 1) / 4 * NDB, "an exp unit would follow its PV MFMA");
  constexpr int NPC = 2 * NKB;    // 8-score pieces of the next tile's max

  // One iteration; sc holds tile t's exp2-domain scores, sn receives tile
  // t+1's.  The loop below alternates the two arrays so that nothing is
  // copied between iterations.
  auto step = [&](int t, f32x16 (&sc)[NKB], f32x16 (&sn)[NKB], u32x4 (&kr)[KLD], u32x4 (&vr)[VLD]) {
    // every wave is done reading K(t) and V(t-1); K(t+1), V(t) are visible
    lds_barrier();
    u32x4 kf[NKB][NKS];
    read_kf(t + 1, kf);  // stale data on the last tile; those scores are dropped
    // this iteration's register set holds K(t+2), V(t+1) (loaded two
    // iterations ago) and is refilled with K(t+4), V(t+3).  Past the last
    // tile the set holds a clamped copy that lands in a buffer no later
    // iteration reads, so the stores need no condition.
    store_k(t + 2, kr);
    store_v(t + 1, vr);
    load_k(t + 4, kr);
    load_v(t + 3, vr);

    // Raise the offset to the row max mx (never lower it once a live key was
    // seen) and rescale O and l; returns the shift applied to the scores.
    auto rescale = [&](float mx) {
      const bool fst = thr == -INFINITY;
      float delta = fst ? mx : fmaxf(mx, 0.f);
      if (mx == -INFINITY) delta = 0.f;
      const float alpha = fast_exp2(-delta);
      mb += delta;
      ls0 *= alpha;
      ls1 *= alpha;
#pragma unroll
      for (int db = 0; db < NDB; ++db) oacc[db] *= alpha;
      if (PRESCALE) bias -= delta;  // stays exactly -mb
      if (!(fst && mx == -INFINITY)) thr = 8.f;
      return delta;
    };

    // ---- rescale decision for tile t: the row max exceeds the offset by
    // more than 8 (log2 units), or this is the first live tile
    {
      const float mx = xhalf_max(mq);
      if (__builtin_amdgcn_ballot_w64(mx > thr)) {
        const float delta = rescale(mx);
#pragma unroll
        for (int kb = 0; kb < NKB; ++kb) sc[kb] -= delta;
      }
    }

    // ---- one basic block, issued in a fixed order (sched_barrier fences):
    // stage A: score MFMAs of tile t+1, each beside V fragment reads of
    // tile t and a share of tile t's exp units; stage B: PV MFMAs of tile
    // t beside the remaining exp units and the pieces of tile t+1's max.
    if (OPT & 1) __builtin_amdgcn_s_setprio(1);
    u32x4 pf[NCH];
    u32x4 vfr[NPV];
    const uint16_t* vs = vbase + (t & 1) * VTILE;
    auto exp_unit = [&](int u) {
      const int ch = u >> 2, e = u & 3, kb = ch >> 1, cc = ch & 1;
      const uint32_t w = Elt<T>::pack(fast_exp2(sc[kb][8 * cc + 2 * e]), fast_exp2(sc[kb][8 * cc + 2 * e + 1]));
      pf[ch][e] = w;
      if (e & 1) ls1 = Elt<T>::sum2(w, ls1);
      else ls0 = Elt<T>::sum2(w, ls0);
    };
    auto read_vfr = [&](int i) {
      const int ch = i / NDB, db = i - ch * NDB;
      const uint16_t* vp = vs + 16 * ch * RSV;
      const uint2 lo = lds_tr16_b64(vp + v_rd[db][0]);
      const uint2 hi = lds_tr16_b64(vp + v_rd[db][1]);
      vfr[i] = (u32x4){lo.x, lo.y, hi.x, hi.y};
    };
    f32x16 acc[NKB];
#pragma unroll
    for (int i = 0; i < NQK; ++i) {
      const int kb = i / NKS, s = i - kb * NKS;
#pragma unroll
      for (int v = i * NPV / NQK; v < (i + 1) * NPV / NQK; ++v) read_vfr(v);
      acc[kb] = Elt<T>::mma(kf[kb][s], qf[s], s == 0 ? (PRESCALE ? bias : (f32x16){}) : acc[kb]);
#pragma unroll
      for (int u = i * UA / NQK; u < (i + 1) * UA / NQK; ++u) exp_unit(u);
      if (!(OPT & 4)) __builtin_amdgcn_sched_barrier(0);
    }

    float mpart = -INFINITY;
    auto piece = [&](int j) {  // 8 scores of the next tile: scale, then max
      const int kb = j >> 1, r0 = 8 * (j & 1);
#pragma unroll
      for (int r = r0; r < r0 + 8; ++r) {
        float x = acc[kb][r];
        if (!PRESCALE) x = __builtin_fmaf(x, c, -mb);
        acc[kb][r] = x;
        mpart = fmaxf(mpart, x);
      }
    };
#pragma unroll
    for (int i = 0; i < NPV; ++i) {
      const int ch = i / NDB, db = i - ch * NDB;
      oacc[db] = Elt<T>::mma(vfr[i], pf[ch], oacc[db]);
      if (i < NU - UA) exp_unit(UA + i);
      else if (i - (NU - UA) < NPC) piece(i - (NU - UA));
      if (!(OPT & 4)) __builtin_amdgcn_sched_barrier(0);
    }
#pragma unroll
    for (int j = NPV - (NU - UA) > 0 ? NPV - (NU - UA) : 0; j < NPC; ++j) piece(j);
    if (OPT & 1) __builtin_amdgcn_s_setprio(0);
    mq = mpart;
#pragma unroll
    for (int kb = 0; kb < NKB; ++kb) sn[kb] = acc[kb];


    if (t + 1 < nt2 && tile_needs_mask(t + 1)) {
      mask(t + 1, sn);
      mq = row_max(sn);
    }
  };

  // An even number of iterations keeps the loop body free of a mid-loop
  // exit, which would make the compiler wait for every prefetch at the top.
  // With an odd tile count the extra tile is a clamped copy of the last one
  // whose keys all lie past kend: fully masked, it adds exactly zero.
  for (int t = 0; t < nt2; t += 2) {
    step(t, sA, sB, kA, vA);
    step(t + 1, sB, sA, kB, vB);
  }

  // ---- epilogue: combine the two halves' partial sums, normalise, store
  const float inv = 1.f / xhalf_sum(ls0 + ls1);
  if (qrow < Sq) {
    uint16_t* orow = og + (int64_t)qrow * p.o_s;
#pragma unroll
    for (int db = 0; db < NDB; ++db)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int d = 32 * db + 8 * g + 4 * hh;
        if (d < D) {
          u32x2 w;
          w[0] = Elt<T>::pack(oacc[db][4 * g + 0] * inv, oacc[db][4 * g + 1] * inv);
          w[1] = Elt<T>::pack(oacc[db][4 * g + 2] * inv, oacc[db][4 * g + 3] * inv);
          *(u32x2*)(orow + d) = w;
        }
      }
  }
}

template <typename T, int DK, int NW, int BK, int OCC, bool CAUSAL, bool PRESCALE, int OPT = 0>
hipError_t launch_pipe16_cfg(const FwdParams& p0, hipStream_t stream) {
  constexpr int DP = (DK + 31) / 32 * 32;
  constexpr int BQ = NW * 32;
  FwdParams p = p0;
  p.n_qblk = (p.Sq + BQ - 1) / BQ;
  p.n_wg = p.B * p.H * p.n_qblk;
  if (p.n_wg == 0) return hipSuccess;
  // buffer offsets of the K/V tiles are 32-bit
  const int64_t rs = p.k_s > p.v_s ? p.k_s : p.v_s;
  if ((int64_t)(p.Sk + BK) * rs * 2 >= (int64_t(1) << 31)) return hipErrorInvalidValue;
  hipLaunchKernelGGL((attn_fwd_pipe16<T, DK, DP, NW, BK, OCC, CAUSAL, PRESCALE, OPT>), dim3(p.n_wg),
                     dim3(NW * 64), 0, stream, p);
  return hipGetLastError();
}

}  // namespace cmpext3
