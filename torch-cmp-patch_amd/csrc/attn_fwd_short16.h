// Fused attention forward for short key sweeps (Sk <= 32 * NKB, NKB <= 4),
// fp16 / bf16 on gfx950 (v_mfma_f32_32x32x16_{f16,bf16}).
//
// SDXL cross-attention (77 text tokens against 4096 image rows) moves 21 MB
// per launch and does little arithmetic, so it is bound by HBM and by the
// latency of each workgroup's load -> compute -> store chain.  Here the whole
// K and V of a (batch, head) fit in LDS: a workgroup issues its Q loads and
// all K/V loads at once, stores K/V to LDS once, meets one barrier, and then
// each wave does its 32 query rows in one pass: every score of the row at
// once (S^T = K Q^T, lane = query row), the exact row max (no running offset,
// no rescale), exponentials, and O^T = V^T P^T, then one store.  Register
// layout, bit-permuted K feed and ds_read_b64_tr_b16 V fragments as in
// attn_fwd_pipe16.h.
//
// Reference algorithm: src/cuda/fp16_flash_attention_hfma2.cu:72-243.
#pragma once

#include "attn_fwd_pipe16.h"

namespace cmpext3 {

// OPT bit 0: s_setprio(1) around the MFMAs.  OPT bit 3: D < DK, K columns past
// D are zeroed (Q is zero there, and 0 * finite keeps the padded k-steps exact).
// NKH: 16-key slices that can hold keys (Sk <= 16 * NKH); the scores come in
// blocks of 32 keys (NKB = ceil(NKH / 2)), but exponentials and PV MFMAs of a
// slice past NKH are skipped (Sk = 77: 5 of 6 slices).
template <typename T, int DK, int DP, int NKH, int OPT = 0>
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu((NKH + 1) / 2 <= 2 ? 3 : 2)))
attn_fwd_short16(const FwdParams p) {
  constexpr int NKB = (NKH + 1) / 2;
  constexpr int NW = 4, NT = 256, BQ = 128;
  constexpr int SK = 32 * NKB;             // keys held (padded)
  constexpr int RSK = DK + 8, RSV = DP + 8;
  constexpr int KCH = DK / 8, VCH = DP / 8;
  constexpr int KLD = (SK * KCH + NT - 1) / NT;
  constexpr int VLD = (SK * VCH + NT - 1) / NT;
  constexpr bool KFULL = SK * KCH % NT == 0;
  constexpr bool VFULL = SK * VCH % NT == 0;
  constexpr int NCH = NKH;                 // 16-key PV slices that hold keys
  constexpr int NDB = DP / 32;
  constexpr int NKS = DK / 16;
  static_assert(NKH >= 1 && NKH <= 8 && DK % 16 == 0 && DP % 32 == 0 && DK <= DP, "tile shape");

  constexpr int RSQ = DP + 8;              // Q / O staging row stride (halves)
  constexpr int QLD = 32 * KCH / 64;       // 16-byte Q chunks per lane (32 rows per wave)
  constexpr int OLD = 32 * VCH / 64;       // 16-byte O chunks per lane
  __shared__ __attribute__((aligned(16))) uint16_t lds[SK * RSK + SK * RSV + NW * 32 * RSQ];
  uint16_t* const ks = lds;
  uint16_t* const vs = lds + SK * RSK;

  const int tid = thread_x(), wave = tid >> 6, lane = tid & 63, l32 = lane & 31, hh = lane >> 5;
  int bh, qblk;
  wg_tile(block_x(), p, false, bh, qblk);
  const int b = bh / p.H, h = bh - b * p.H;
  const int Sq = p.Sq, Sk = p.Sk, D = p.D;
  const int qlo = qblk * BQ + wave * 32;   // first query row of this wave
  // this wave's staging rows: Q on the way in, O on the way out, so that both
  // global transfers are whole 16-byte chunks of consecutive memory per lane
  uint16_t* const qs = lds + SK * RSK + SK * RSV + wave * 32 * RSQ;

  const uint16_t* __restrict__ qg = (const uint16_t*)p.q + b * p.q_b + h * p.q_h;
  const uint16_t* kg = (const uint16_t*)p.k + b * p.k_b + (h / p.kv_group) * p.k_h;
  const uint16_t* vg = (const uint16_t*)p.v + b * p.v_b + (h / p.kv_group) * p.v_h;
  uint16_t* __restrict__ og = (uint16_t*)p.o + b * p.o_b + h * p.o_h;

  // ---- every global load first: this wave's 32 Q rows in row order (chunk
  // i of the 32 x KCH chunks to lane i mod 64), then all of K/V.  All of them
  // are buffer accesses over this (batch, head)'s rows with 32-bit offsets
  // (the host checks the extent): rows at or past Sq / Sk read as zero and O
  // stores past Sq are dropped, so no row needs a condition.  When the chunks
  // of a row divide the lanes, a load's row step is a scalar offset.
  const int qs_b = (int)p.q_s * 2, os_b = (int)p.o_s * 2;
  const int ks_b = (int)p.k_s * 2, vs_b = (int)p.v_s * 2;
  const __amdgpu_buffer_rsrc_t qrs = uniform_rsrc(qg, ((int64_t)(Sq - 1) * p.q_s + D) * 2);
  const __amdgpu_buffer_rsrc_t ors = uniform_rsrc(og, ((int64_t)(Sq - 1) * p.o_s + D) * 2);
  const __amdgpu_buffer_rsrc_t krs = uniform_rsrc(kg, ((int64_t)(Sk - 1) * p.k_s + D) * 2);
  const __amdgpu_buffer_rsrc_t vrs = uniform_rsrc(vg, ((int64_t)(Sk - 1) * p.v_s + D) * 2);
  // byte offset of 16-byte chunk i (of NCHK per row) within rows of rb bytes:
  // lane part in the vector offset, row step of iteration it in the scalar one
  auto chunk_off = [](int i, int it, int per_it, int nchk, int rb, int& vo, int& so) {
    if (per_it % nchk == 0) {
      const int r = i / nchk;
      vo = r * rb + 16 * (i - r * nchk);
      so = it * (per_it / nchk) * rb;
    } else {
      const int ci = it * per_it + i, r = ci / nchk;
      vo = r * rb + 16 * (ci - r * nchk);
      so = 0;
    }
  };
  u32x4 qr[QLD];
#pragma unroll
  for (int it = 0; it < QLD; ++it) {
    int vo, so;
    chunk_off(lane, it, 64, KCH, qs_b, vo, so);
    u32x4 x = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(qrs, qlo * qs_b + vo, so, 0));
    const int c8 = (it * 64 + lane) % KCH;
    if ((OPT & 8) && 8 * c8 >= D) x = (u32x4){0u, 0u, 0u, 0u};  // the next row's head dims
    qr[it] = x;
  }
  u32x4 kr[KLD], vr[VLD];
#pragma unroll
  for (int it = 0; it < KLD; ++it) {
    int vo, so;
    chunk_off(tid, it, NT, KCH, ks_b, vo, so);
    kr[it] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(krs, vo, so, 0));
  }
#pragma unroll
  for (int it = 0; it < VLD; ++it) {
    int vo, so;
    chunk_off(tid, it, NT, VCH, vs_b, vo, so);
    vr[it] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(vrs, vo, so, 0));
  }
#pragma unroll
  for (int it = 0; it < KLD; ++it) {
    const int ci = it * NT + tid, r = ci / KCH, c8 = ci - r * KCH;
    if (KFULL || ci < SK * KCH) {
      u32x4 x = kr[it];
      if ((OPT & 8) && 8 * c8 >= D) x = (u32x4){0u, 0u, 0u, 0u};
      *(u32x4*)(ks + r * RSK + 8 * c8) = x;
    }
  }
#pragma unroll
  for (int it = 0; it < VLD; ++it) {
    const int ci = it * NT + tid, r = ci / VCH, c8 = ci - r * VCH;
    if (VFULL || ci < SK * VCH) *(u32x4*)(vs + r * RSV + 8 * c8) = vr[it];
  }
  // Q through this wave's staging rows into the B-operand layout (lane = row,
  // 8 head-dim values per k-step); LDS accesses of one wave stay in order
#pragma unroll
  for (int it = 0; it < QLD; ++it) {
    const int ci = it * 64 + lane, r = ci / KCH, c8 = ci - r * KCH;
    *(u32x4*)(qs + r * RSQ + 8 * c8) = qr[it];
  }
  u32x4 qf[NKS];
#pragma unroll
  for (int s = 0; s < NKS; ++s) qf[s] = *(const u32x4*)(qs + l32 * RSQ + 16 * s + 8 * hh);
  if (p.q_sign) {  // negative scale (uniform)
#pragma unroll
    for (int s = 0; s < NKS; ++s) qf[s] ^= p.q_sign;
  }
  lds_barrier();

  // ---- all scores of the row: S^T = K Q^T over NKB blocks of 32 keys
  if (OPT & 1) __builtin_amdgcn_s_setprio(1);
  f32x16 sc[NKB];
  {
    const int r = perm_row(l32);
#pragma unroll
    for (int kb = 0; kb < NKB; ++kb) {
      f32x16 acc = (f32x16){};
#pragma unroll
      for (int s = 0; s < NKS; ++s)
        acc = Elt<T>::mma(*(const u32x4*)(ks + (32 * kb + r) * RSK + 16 * s + 8 * hh), qf[s], acc);
      sc[kb] = acc;
    }
  }
  if (OPT & 1) __builtin_amdgcn_s_setprio(0);

  // ---- exact softmax over the row.  Keys past Sk are masked only in the
  // blocks that reach past it (a uniform branch: the key capacity keeps every
  // block but the last whole when Sk > 48).  The max is taken over the raw
  // scores and the exp2 argument is one FMA, s * c - m * c (c > 0; the host
  // turns scale 0 into a tiny c, so masked keys stay -inf instead of 0 * inf).
  const float c = p.c;
  float mq = -INFINITY;
#pragma unroll
  for (int kb = 0; kb < NKB; ++kb) {
    if (32 * (kb + 1) > Sk) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        if (2 * kb + (r >> 3) >= NKH) continue;  // a slice past every key
        if (32 * kb + acc_key(r, hh) >= Sk) sc[kb][r] = -INFINITY;
      }
    }
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      if (2 * kb + (r >> 3) >= NKH) continue;
      mq = fmaxf(mq, sc[kb][r]);
    }
  }
  const float m = xhalf_max(mq) * c;  // finite: Sk >= 1 keeps key 0 in every row
  u32x4 pf[NCH];
  float ls0 = 0.f, ls1 = 0.f;
#pragma unroll
  for (int ch = 0; ch < NCH; ++ch)
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int kb = ch >> 1, cc = ch & 1;
      const uint32_t w = Elt<T>::pack(fast_exp2(__builtin_fmaf(sc[kb][8 * cc + 2 * e], c, -m)),
                                      fast_exp2(__builtin_fmaf(sc[kb][8 * cc + 2 * e + 1], c, -m)));
      pf[ch][e] = w;
      if (e & 1) ls1 = Elt<T>::sum2(w, ls1);
      else ls0 = Elt<T>::sum2(w, ls0);
    }

  // ---- O^T = V^T P^T
  const int jj = lane & 15, gg = lane >> 4;
  int v_rd[NDB][2];
#pragma unroll
  for (int db = 0; db < NDB; ++db)
#pragma unroll
    for (int half = 0; half < 2; ++half)
      v_rd[db][half] = (8 * (gg >> 1) + (jj >> 2) + 4 * half) * RSV + 32 * db + 16 * (gg & 1) + 4 * (jj & 3);
  if (OPT & 1) __builtin_amdgcn_s_setprio(1);
  f32x16 oacc[NDB];
#pragma unroll
  for (int db = 0; db < NDB; ++db) oacc[db] = (f32x16){};
#pragma unroll
  for (int ch = 0; ch < NCH; ++ch)
#pragma unroll
    for (int db = 0; db < NDB; ++db) {
      const uint16_t* vp = vs + 16 * ch * RSV;
      const uint2 lo = lds_tr16_b64(vp + v_rd[db][0]);
      const uint2 hi = lds_tr16_b64(vp + v_rd[db][1]);
      oacc[db] = Elt<T>::mma((u32x4){lo.x, lo.y, hi.x, hi.y}, pf[ch], oacc[db]);
    }
  if (OPT & 1) __builtin_amdgcn_s_setprio(0);

  // ---- O rows through the staging rows (the wave read its Q from them
  // already), then whole 16-byte chunks out
  const float inv = 1.f / xhalf_sum(ls0 + ls1);
#pragma unroll
  for (int db = 0; db < NDB; ++db)
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      u32x2 w;
      w[0] = Elt<T>::pack(oacc[db][4 * g + 0] * inv, oacc[db][4 * g + 1] * inv);
      w[1] = Elt<T>::pack(oacc[db][4 * g + 2] * inv, oacc[db][4 * g + 3] * inv);
      *(u32x2*)(qs + l32 * RSQ + 32 * db + 8 * g + 4 * hh) = w;
    }
#pragma unroll
  for (int it = 0; it < OLD; ++it) {
    const int ci = it * 64 + lane, r = ci / VCH, c8 = ci - r * VCH;
    const u32x4 x = *(const u32x4*)(qs + r * RSQ + 8 * c8);
    int vo, so;
    chunk_off(lane, it, 64, VCH, os_b, vo, so);
    // chunks past D (a head dim below its bucket, or DP > DK) would land on
    // the next row's head dims
    if (!((OPT & 8) || DP != DK) || 8 * c8 < D)
      __builtin_amdgcn_raw_buffer_store_b128(x, ors, qlo * os_b + vo, so, 0);
  }
}

template <typename T, int DK, int NKH, int OPT = 0>
hipError_t launch_short16_cfg(const FwdParams& p0, hipStream_t stream) {
  constexpr int NKB = (NKH + 1) / 2;
  constexpr int DP = (DK + 31) / 32 * 32;
  FwdParams p = p0;
  if (p.c == 0.f) p.c = 1e-30f;  // scale 0: every finite exp2 argument rounds to 0
  p.n_qblk = (p.Sq + 127) / 128;
  p.n_wg = p.B * p.H * p.n_qblk;
  if (p.n_wg == 0) return hipSuccess;
  const int64_t rs = p.k_s > p.v_s ? p.k_s : p.v_s;
  if ((int64_t)(32 * NKB) * rs * 2 >= (int64_t(1) << 31)) return hipErrorInvalidValue;
  if (p.dry) return hipSuccess;  // never splits
  hipLaunchKernelGGL((attn_fwd_short16<T, DK, DP, NKH, OPT>), dim3(p.n_wg), dim3(256), 0, stream, p);
  return hipGetLastError();
}

}  // namespace cmpext3
