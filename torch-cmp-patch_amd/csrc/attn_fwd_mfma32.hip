// Fused attention forward for fp32 on gfx950 fp32 MFMA (v_mfma_f32_16x16x4f32).
//
// Same structure as the fp16/bf16 kernel (one workgroup = one (batch, head)
// pair x BQ query rows; K/V tiles double-buffered through LDS; S^T = K Q^T so
// that each lane owns one query column), but on 16x16 fp32 MFMA blocks: the
// products are exact fp32 products accumulated in fp32, so no precision is
// given up anywhere (the north-star bound for fp32 is 1e-4 max abs error).
// In the 16x16 accumulator a lane holds 4 consecutive keys of one query, so a
// row reduction spans the 4 lane groups (two cross-lane steps), and P^T feeds
// the PV MFMA's B operand one accumulator element per k-step, lane-local.
// V stays row-major in LDS: a PV A-operand element is V[key][d] with d along
// the 16 lanes of a group, which is a conflict-free LDS read.
//
// With p.lse set (the training forward) each row's natural-log log-sum-exp
// is written too (by the merging part where the keys are split: the merged
// offset and row sum).
//
// Key split (launches with at most as many query blocks as CUs, such as
// [1, 8, 1024, 64]; causal ones where most CUs idle or sweeps are long): each
// block's key range is cut into parts run by
// separate workgroups, which shortens every wave's dependency chain over the
// keys and fills the idle CUs.  Every part leaves its fp32 (O, m, l) in the exchange
// buffer; the last part of a (block, wave) to finish merges all of them in
// part order and writes the output (the many-part protocol of
// attn_fwd_pipe16.h).
//
// Reference: src/cuda/fp32_attention.cu:35-198 (one thread per query row,
// serial D loops, non-causal only, Sq == Sk only, D <= 128, and 1/l taken
// through an fp16 reciprocal at :179-180).  This kernel drops every one of
// those limits; 1/l is an fp32 reciprocal.
#include "attn_common.h"

namespace cmpext3 {

__device__ __forceinline__ f32x4 mma32(float a, float b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

// DK: head dim bucket (multiple of 4, zero-padded above D); NQB: 16-row query
// blocks per wave.  ELEM: element-granular K/V/O rows (any head dim, any
// 4-byte aligned rows; ld_cols32), columns past D never touched.  MASK: an
// attention mask (p.mask: bool keeps, floats are added to the scaled scores)
// applied to every tile.
template <int DK, int NW, int NQB, int BK, bool CAUSAL, bool ELEM, bool MASK = false>
__global__ void __launch_bounds__(NW * 64)
attn_fwd_mfma32(const FwdParams p, const SplitArgs sa) {
  constexpr int NT = NW * 64;
  constexpr int QPW = 16 * NQB;
  constexpr int BQ = NW * QPW;
  constexpr int DPV = (DK + 15) / 16 * 16;                  // PV output rows
  constexpr int RSK = ((DK / 4) % 2 == 0) ? DK + 4 : DK;    // 4*odd floats: conflict-free
  constexpr int RSV = DPV + 4;                              // 4 mod 16 floats
  constexpr int KTILE = BK * RSK;
  constexpr int VTILE = BK * RSV;
  constexpr int KCH = DK / 4;       // 16-byte chunks per K row
  constexpr int VCH = DPV / 4;
  constexpr int KLD = (BK * KCH + NT - 1) / NT;
  constexpr int VLD = (BK * VCH + NT - 1) / NT;
  constexpr int NKB = BK / 16;
  constexpr int NDB = DPV / 16;
  constexpr int NKS = DK / 4;
  static_assert(BK % 16 == 0 && DK % 4 == 0, "tile shape");

  __shared__ __attribute__((aligned(16))) float lds[2 * (KTILE + VTILE)];

  const int tid = thread_x();
  const int wave = tid >> 6;
  const int lane = tid & 63;
  const int l16 = lane & 15;
  const int g = lane >> 4;

  int lb = block_x(), part = 0, nparts = 1;
  if (lb >= sa.nfull) {
    const int r = lb - sa.nfull;
    nparts = sa.nparts;
    lb = sa.nfull + r / nparts;
    part = r - (lb - sa.nfull) * nparts;
  }
  int bh, qblk;
  wg_tile(lb, p, CAUSAL, bh, qblk);
  const int b = bh / p.H;
  const int h = bh - b * p.H;
  const int q0 = qblk * BQ;

  const float* __restrict__ qg = (const float*)p.q + b * p.q_b + h * p.q_h;
  const float* __restrict__ kg = (const float*)p.k + b * p.k_b + (h / p.kv_group) * p.k_h;
  const float* __restrict__ vg = (const float*)p.v + b * p.v_b + (h / p.kv_group) * p.v_h;
  float* __restrict__ og = (float*)p.o + b * p.o_b + h * p.o_h;

  const int Sq = p.Sq, Sk = p.Sk, D = p.D;
  const int qw0 = q0 + wave * QPW;

  int kend = Sk;
  if (CAUSAL) kend = min(Sk, q0 + BQ);
  // this workgroup's key tiles [tbase, tbase + ntiles)
  const int ntall = (kend + BK - 1) / BK;
  const int tbase = part * ntall / nparts;
  const int ntiles = (part + 1) * ntall / nparts - tbase;

  // Q^T as the B operand: lane (l16, g) holds Q[row][4s + g]
  float qf[NQB][NKS];
  const float qsign = p.q_sign ? -1.f : 1.f;
#pragma unroll
  for (int qb = 0; qb < NQB; ++qb) {
    const int row = qw0 + 16 * qb + l16;
#pragma unroll
    for (int s = 0; s < NKS; ++s) {
      const int d = 4 * s + g;
      qf[qb][s] = (row < Sq && d < D) ? qsign * qg[(int64_t)row * p.q_s + d] : 0.f;
    }
  }

  f32x4 oacc[NQB][NDB];
#pragma unroll
  for (int qb = 0; qb < NQB; ++qb)
#pragma unroll
    for (int db = 0; db < NDB; ++db) oacc[qb][db] = (f32x4){};
  float m_run[NQB], l_run[NQB];
#pragma unroll
  for (int qb = 0; qb < NQB; ++qb) {
    m_run[qb] = -INFINITY;
    l_run[qb] = 0.f;
  }
  const float c = p.c;

  u32x4 kreg[KLD], vreg[VLD];
  auto load_tile = [&](int t) {
    const int k0 = (tbase + t) * BK;
#pragma unroll
    for (int it = 0; it < KLD; ++it) {
      const int ci = it * NT + tid;
      const int r = ci / KCH, c4 = ci - (ci / KCH) * KCH;
      u32x4 x = {0u, 0u, 0u, 0u};
      if ((BK * KCH % NT == 0 || ci < BK * KCH) && k0 + r < Sk && 4 * c4 < D) {
        const float* src = kg + (int64_t)(k0 + r) * p.k_s + 4 * c4;
        x = ELEM ? ld_cols32(src, D - 4 * c4) : *(const u32x4*)src;
      }
      kreg[it] = x;
    }
#pragma unroll
    for (int it = 0; it < VLD; ++it) {
      const int ci = it * NT + tid;
      const int r = ci / VCH, c4 = ci - (ci / VCH) * VCH;
      u32x4 x = {0u, 0u, 0u, 0u};
      if ((BK * VCH % NT == 0 || ci < BK * VCH) && k0 + r < Sk && 4 * c4 < D) {
        const float* src = vg + (int64_t)(k0 + r) * p.v_s + 4 * c4;
        x = ELEM ? ld_cols32(src, D - 4 * c4) : *(const u32x4*)src;
      }
      vreg[it] = x;
    }
  };
  // K rows in LDS: the two 8-byte halves of every 16-byte chunk trade places
  // in rows 8-15 of each 16.  A 4-byte K fragment read serves 32 lanes (16
  // rows x lane groups g = 0, 1, or 2, 3) per pass over 32 banks; with a row
  // stride of 4 * odd floats, rows l and l + 8 start on the same bank, and
  // the swap moves row l + 8's two lane groups to the other two banks of
  // each 4-bank group (without it K reads took two passes; measured
  // SQ_LDS_BANK_CONFLICT ~28-30% of LDS cycles).
  auto store_tile = [&](int buf) {
    float* ks = lds + buf * (KTILE + VTILE);
    float* vs = ks + KTILE;
#pragma unroll
    for (int it = 0; it < KLD; ++it) {
      const int ci = it * NT + tid;
      if (BK * KCH % NT == 0 || ci < BK * KCH) {
        const int r = ci / KCH, c4 = ci - (ci / KCH) * KCH;
        const u32x4 x = kreg[it];
        *(u32x4*)(ks + r * RSK + 4 * c4) = (r & 8) ? (u32x4){x[2], x[3], x[0], x[1]} : x;
      }
    }
#pragma unroll
    for (int it = 0; it < VLD; ++it) {
      const int ci = it * NT + tid;
      if (BK * VCH % NT == 0 || ci < BK * VCH) {
        const int r = ci / VCH, c4 = ci - (ci / VCH) * VCH;
        *(u32x4*)(vs + r * RSV + 4 * c4) = vreg[it];
      }
    }
  };

  // attention mask rows (MASK): rows past Sq read the last row (their output
  // is never stored); the (batch, head)'s mask is readable up to key Sk - 1
  // of its last row (a narrow mask, read element by element) or up to Sk
  // rounded up to 8; reads past that return zero, and keys at or past Sk are
  // masked by the key-range rule anyway
  const int mes = p.mask_kind == MASK_BOOL ? 1 : p.mask_kind == MASK_F32 ? 4 : 2;
  const __amdgpu_buffer_rsrc_t mrs =
      uniform_rsrc(MASK ? (const void*)((const char*)p.mask + (b * p.m_b + h * p.m_h) * mes) : p.q,
                   MASK ? ((int64_t)(Sq - 1) * p.m_q + (p.mask_narrow ? Sk : (Sk + 7) / 8 * 8)) * mes : 0);
  int mrow[NQB];
#pragma unroll
  for (int qb = 0; qb < NQB; ++qb)
    mrow[qb] = MASK ? (int)((int64_t)min(qw0 + 16 * qb + l16, Sq - 1) * p.m_q * mes) : 0;

  if (ntiles > 0) load_tile(0);

  for (int t = 0; t < ntiles; ++t) {
    const int buf = t & 1;
    store_tile(buf);
    __syncthreads();
    if (t + 1 < ntiles) load_tile(t + 1);

    const int k0 = (tbase + t) * BK;
    const bool active = !CAUSAL || k0 <= qw0 + QPW - 1;
    if (active) {
      const float* ks = lds + buf * (KTILE + VTILE);
      const float* vs = ks + KTILE;

      f32x4 sacc[NQB][NKB];
#pragma unroll
      for (int kb = 0; kb < NKB; ++kb) {
#pragma unroll
        for (int qb = 0; qb < NQB; ++qb) sacc[qb][kb] = (f32x4){};
        const float* krow = ks + (16 * kb + l16) * RSK + (g ^ ((l16 >> 2) & 2));
        if (!CAUSAL) __builtin_amdgcn_s_setprio(1);
#pragma unroll
        for (int s = 0; s < NKS; ++s) {
          const float a = krow[4 * s];
#pragma unroll
          for (int qb = 0; qb < NQB; ++qb) sacc[qb][kb] = mma32(a, qf[qb][s], sacc[qb][kb]);
        }
        if (!CAUSAL) __builtin_amdgcn_s_setprio(0);
      }

      const bool need_mask = MASK || (k0 + BK > Sk) || (CAUSAL && k0 + BK - 1 > qw0);
      float cm = c;
      if (need_mask) {
#pragma unroll
        for (int qb = 0; qb < NQB; ++qb) {
          const int qrow = qw0 + 16 * qb + l16;
#pragma unroll
          for (int kb = 0; kb < NKB; ++kb) {
            // the lane's 4 consecutive keys: one 4/8/16-byte mask read
            f32x4 madd = {0.f, 0.f, 0.f, 0.f};
            uint32_t keep = 0x01010101u;
            if (MASK && p.mask_narrow) {
              const int key4 = k0 + 16 * kb + 4 * g;
#pragma unroll
              for (int r = 0; r < 4; ++r) {
                const int off = mrow[qb] + (key4 + r) * mes;
                if (p.mask_kind == MASK_BOOL) {
                  if (__builtin_amdgcn_raw_buffer_load_b8(mrs, off, 0, 0) == 0) keep &= ~(0xffu << (8 * r));
                } else if (p.mask_kind == MASK_F32) {
                  madd[r] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(mrs, off, 0, 0));
                } else {
                  const uint32_t hb = __builtin_amdgcn_raw_buffer_load_b16(mrs, off, 0, 0);
                  madd[r] = p.mask_kind == MASK_F16 ? (float)__builtin_bit_cast(_Float16, (uint16_t)hb)
                                                    : __uint_as_float(hb << 16);
                }
              }
            } else if (MASK) {
              const int key4 = k0 + 16 * kb + 4 * g;
              if (p.mask_kind == MASK_BOOL) {
                keep = __builtin_amdgcn_raw_buffer_load_b32(mrs, mrow[qb] + key4, 0, 0);
              } else if (p.mask_kind == MASK_F32) {
                madd = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(mrs, mrow[qb] + 4 * key4, 0, 0));
              } else {
                const u32x2 w = __builtin_bit_cast(u32x2, __builtin_amdgcn_raw_buffer_load_b64(mrs, mrow[qb] + 2 * key4, 0, 0));
#pragma unroll
                for (int i = 0; i < 2; ++i) {
                  const uint32_t lo = w[i] << 16, hi = w[i] & 0xffff0000u;
                  if (p.mask_kind == MASK_BF16) {
                    madd[2 * i] = __uint_as_float(lo);
                    madd[2 * i + 1] = __uint_as_float(hi);
                  } else {
                    madd[2 * i] = (float)__builtin_bit_cast(_Float16, (uint16_t)(w[i] & 0xffffu));
                    madd[2 * i + 1] = (float)__builtin_bit_cast(_Float16, (uint16_t)(w[i] >> 16));
                  }
                }
              }
            }
#pragma unroll
            for (int r = 0; r < 4; ++r) {
              const int key = k0 + 16 * kb + 4 * g + r;
              const bool dead = key >= Sk || (CAUSAL && key > qrow) || ((keep >> (8 * r)) & 0xffu) == 0u;
              sacc[qb][kb][r] = dead ? -INFINITY : __builtin_fmaf(madd[r], kLog2e, sacc[qb][kb][r] * c);
            }
          }
        }
        cm = 1.f;
      }

      float pr[NQB][NKB][4];
#pragma unroll
      for (int qb = 0; qb < NQB; ++qb) {
        float mx = -INFINITY;
#pragma unroll
        for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
          for (int r = 0; r < 4; ++r) mx = fmaxf(mx, sacc[qb][kb][r]);
        mx = fmaxf(mx, __shfl_xor(mx, 16));
        mx = fmaxf(mx, __shfl_xor(mx, 32));
        const float m_tile = (mx == -INFINITY) ? -INFINITY : mx * cm;
        const float m_new = fmaxf(m_run[qb], m_tile);
        const float m_use = (m_new == -INFINITY) ? 0.f : m_new;
        const float alpha = fast_exp2(m_run[qb] - m_use);
        m_run[qb] = m_new;
        float lsum = l_run[qb] * alpha;
#pragma unroll
        for (int db = 0; db < NDB; ++db) oacc[qb][db] *= alpha;
#pragma unroll
        for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const float pv = fast_exp2(sacc[qb][kb][r] * cm - m_use);
            pr[qb][kb][r] = pv;
            lsum += pv;
          }
        l_run[qb] = lsum;
      }

      // O^T += V^T P^T, one 4-key k-slice per (kb, r).  Non-causal launches
      // raise the wave's issue priority around their MFMA blocks (1-2% on
      // MI355X, [2,8,4096,4096,40] and D = 64); causal ones lose 3-7% with it.
      if (!CAUSAL) __builtin_amdgcn_s_setprio(1);
#pragma unroll
      for (int db = 0; db < NDB; ++db) {
#pragma unroll
        for (int kb = 0; kb < NKB; ++kb) {
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const float a = vs[(16 * kb + 4 * g + r) * RSV + 16 * db + l16];
#pragma unroll
            for (int qb = 0; qb < NQB; ++qb) oacc[qb][db] = mma32(a, pr[qb][kb][r], oacc[qb][db]);
          }
        }
      }
      if (!CAUSAL) __builtin_amdgcn_s_setprio(0);
    }
  }

  // full row sums (each lane summed its own keys)
  float lrow[NQB];
#pragma unroll
  for (int qb = 0; qb < NQB; ++qb) {
    float l = l_run[qb];
    l += __shfl_xor(l, 16);
    l += __shfl_xor(l, 32);
    lrow[qb] = l;
  }
  if (nparts > 1) {
    // a wave whose rows all lie past Sq has nothing to exchange; every part
    // of the block agrees on that
    if (qw0 >= Sq) return;
    // Every part leaves its state and counts itself in; the last one in
    // merges (its own state straight from registers) and writes the output.
    // Device-scope (aux 16 = sc1) 16-byte accesses, coherent across the
    // XCDs' L2s; fp32 goes through bit casts because the builtins move dwords.
    constexpr int NV = NQB * (NDB + 1);
    const int sb = lb - sa.nfull, nwl = sa.nwl;
    const __amdgpu_buffer_rsrc_t wsr = uniform_rsrc(sa.ws, (int64_t)(sb + 1) * nparts * nwl * NV * 64 * 16);
    auto voff = [&](int q, int k) { return ((((sb * nparts + q) * nwl + wave) * NV + k) * 64 + lane) * 16; };
    auto st_ws = [&](f32x4 x, int off) {
      __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, x), wsr, off, 0, 16);
    };
    auto ld_ws = [&](int off) { return __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(wsr, off, 0, 16)); };
    int* const ctr = sa.cnt + 2 * (sb * nwl + wave);  // parts in (the second counter is unused here)
    // a row whose keys of this part are all masked holds nothing: offset -inf
    float m_own[NQB];
#pragma unroll
    for (int qb = 0; qb < NQB; ++qb) {
      m_own[qb] = lrow[qb] > 0.f ? m_run[qb] : -INFINITY;
#pragma unroll
      for (int db = 0; db < NDB; ++db) st_ws(oacc[qb][db], voff(part, qb * (NDB + 1) + db));
      st_ws((f32x4){m_own[qb], lrow[qb], 0.f, 0.f}, voff(part, qb * (NDB + 1) + NDB));
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    int old = 0;
    if (lane == 0) old = __hip_atomic_fetch_add(ctr, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    old = __builtin_amdgcn_readfirstlane(old);
    if (old != nparts - 1) return;
    if (lane == 0) __hip_atomic_store(ctr, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    asm volatile("" ::: "memory");  // the exchange loads stay after the count
    // merge in part order, this part from its registers: the same
    // instructions on the same values whichever part arrives last.  The
    // exchange loads of CH parts are issued together (one memory round trip
    // per CH parts instead of one per part); part indices past the last are
    // clamped to it and their values dropped.
    constexpr int CH = 4;
#pragma unroll
    for (int qb = 0; qb < NQB; ++qb) {
      float mt = m_own[qb];
      for (int q0 = 0; q0 < nparts; q0 += CH) {
        float mq[CH];
#pragma unroll
        for (int j = 0; j < CH; ++j) mq[j] = ld_ws(voff(min(q0 + j, nparts - 1), qb * (NDB + 1) + NDB))[0];
#pragma unroll
        for (int j = 0; j < CH; ++j)
          if (q0 + j < nparts && q0 + j != part) mt = fmaxf(mt, mq[j]);
      }
      f32x4 own[NDB];
#pragma unroll
      for (int db = 0; db < NDB; ++db) {
        own[db] = oacc[qb][db];
        oacc[qb][db] = (f32x4){};
      }
      float l = 0.f;
      for (int q0 = 0; q0 < nparts; q0 += CH) {
        f32x4 ml[CH], x[CH][NDB];
#pragma unroll
        for (int j = 0; j < CH; ++j) {
          const int qq = min(q0 + j, nparts - 1);
          ml[j] = ld_ws(voff(qq, qb * (NDB + 1) + NDB));
#pragma unroll
          for (int db = 0; db < NDB; ++db) x[j][db] = ld_ws(voff(qq, qb * (NDB + 1) + db));
        }
#pragma unroll
        for (int j = 0; j < CH; ++j) {
          const int q = q0 + j;
          if (q >= nparts) break;
          const bool mine = q == part;
          const float mq = mine ? m_own[qb] : ml[j][0];
          const float a = mq == -INFINITY ? 0.f : fast_exp2(mq - mt);
          l = __builtin_fmaf(mine ? lrow[qb] : ml[j][1], a, l);
#pragma unroll
          for (int db = 0; db < NDB; ++db)
#pragma unroll
            for (int i = 0; i < 4; ++i)
              oacc[qb][db][i] = __builtin_fmaf(mine ? own[db][i] : x[j][db][i], a, oacc[qb][db][i]);
        }
      }
      lrow[qb] = l;
      m_run[qb] = mt;  // the merged offset, for the log-sum-exp
    }
  }

#pragma unroll
  for (int qb = 0; qb < NQB; ++qb) {
    // a row that saw no key at all gives zeros, as torch does
    const float inv = lrow[qb] > 0.f ? 1.f / lrow[qb] : 0.f;
    const int qrow = qw0 + 16 * qb + l16;
    // training forward: log-sum-exp in natural log, (m + log2 l) * ln 2
    // (m is the exp2-domain offset, equal in the row's four lane groups);
    // -inf for a row that saw no key
    if (p.lse && qrow < Sq && g == 0)
      p.lse[(int64_t)bh * Sq + qrow] =
          lrow[qb] > 0.f ? (m_run[qb] + __builtin_amdgcn_logf(lrow[qb])) * 0.6931471805599453f : -INFINITY;
    if (qrow < Sq) {
      float* orow = og + (int64_t)qrow * p.o_s;
#pragma unroll
      for (int db = 0; db < NDB; ++db) {
        const int d = 16 * db + 4 * g;
        if (ELEM) {
#pragma unroll
          for (int e = 0; e < 4; ++e)
            if (d + e < D) orow[d + e] = oacc[qb][db][e] * inv;
        } else if (d < D) {
          *(f32x4*)(orow + d) = oacc[qb][db] * inv;
        }
      }
    }
  }
}

// Key split plan: only when the query blocks leave CUs idle or alone (at most
// one block per CU), into enough parts for about two workgroups per CU, each
// part at least kMinTiles32 key tiles long (causal: below).  Returns the part
// count (1: no split) for n query blocks and bk-key tiles.  Measured on
// MI355X at one block per CU (n = 256, 2 parts, 64-key tiles against the
// unsplit launch): [2,8,1024,1024,64] 60.8 -> 54.1 us, [2,8,1024,4096,64]
// 215 -> 172 us, [1,8,2048,2048,40] 95.5 -> 69.2 us, [2,8,1024,1024,128]
// (32-key tiles) 107 -> 101 us; between one and two blocks per CU a split
// changes nothing.
//
// Causal launches (query blocks of 64 rows whose sweeps end at their last
// row): every block is cut into the same number of parts where the blocks
// leave more than half of the CUs idle or sweep long key ranges (the last
// block at least kLongCausal32 tiles), the longest part keeping at least
// kMinCausalTiles32 tiles and every part at least one (a causal row sees a
// key in the first tile of a part or none of its keys; the kernel gives such
// a row's part no weight in the merge).
constexpr int kMinTiles32 = 4;
constexpr int kMinCausalTiles32 = 8;
constexpr int kLongCausal32 = 64;
int split_parts32(int n, int Sk, int bk, int cus, bool causal, int Sq) {
  if (n <= 0 || n > cus) return 1;
  int parts = 2 * cus / n;
  if (causal) {
    const int64_t last = (int64_t)(Sq + 63) / 64 * 64;  // keys the last block's rows can see
    const int tmax = (int)(((last < Sk ? last : Sk) + bk - 1) / bk);
    const int tmin = ((Sk < 64 ? Sk : 64) + bk - 1) / bk;
    if (n * 2 > cus && tmax < kLongCausal32) return 1;
    if (parts > tmax / kMinCausalTiles32) parts = tmax / kMinCausalTiles32;
    if (parts > tmin) parts = tmin;
    if (parts > 8) parts = 8;
    return parts >= 2 ? parts : 1;
  }
  const int ntiles = (Sk + bk - 1) / bk;
  if (parts > ntiles / kMinTiles32) parts = ntiles / kMinTiles32;
  return parts >= 2 ? parts : 1;
}

// Keys per tile: 32 (16 above D = 128).  Head dims up to 64 take 64-key
// tiles, half the barriers per key, in split launches where that keeps the
// part count and in unsplit non-causal launches of one to two blocks per CU,
// all of them resident at the two workgroups per CU that 64-key tiles leave
// room for in LDS (measured on MI355X: [1,8,1024,1024,64], 128 blocks x 4
// parts, 34.1 -> 33.0 us; 320 to 448 unsplit blocks of [B,H,1024,1024,64]
// 93.5-94.9 -> 89.0-91.0 us).  Beyond two blocks per CU 32-key tiles keep
// more workgroups resident: an unsplit [2,8,4096,4096,64] (1024 blocks) takes
// 601 us with 32, 635 with 64.
int tile_keys32(int dk, int n, int Sk, int cus, bool causal) {
  const int def = dk <= 128 ? 32 : 16;
  if (dk > 64 || causal) return def;
  if (!causal && n > cus) return n <= 2 * cus ? 64 : def;
  const int p64 = split_parts32(n, Sk, 64, cus, false, 0);
  return p64 >= 2 && p64 == split_parts32(n, Sk, def, cus, false, 0) ? 64 : def;
}

template <int DK, bool CAUSAL, bool ELEM, int BK, bool MASK>
hipError_t launch_mfma32_bk(const FwdParams& p0, hipStream_t stream) {
  // One 16-row query block per wave: measured on MI355X, two per wave only
  // lengthen each wave's dependency chain (1.6x slower on [1,8,1024,1024,64],
  // 19% slower causal, equal on [2,8,4096,4096,40]), and 64-row workgroups
  // fill more CUs on small grids.
  constexpr int NW = 4;
  constexpr int NQB = 1;
  constexpr int BQ = NW * 16 * NQB;
  constexpr int NDB = (DK + 15) / 16;
  FwdParams p = p0;
  p.n_qblk = (p.Sq + BQ - 1) / BQ;
  p.n_wg = p.B * p.H * p.n_qblk;
  if (p.n_wg == 0) return hipSuccess;
  const int n = p.n_wg;
  // waves per block that hold query rows (a single block shorter than BQ has fewer)
  const int nwl = p.n_qblk > 1 ? NW : (p.Sq + 15) / 16 < NW ? (p.Sq + 15) / 16 : NW;
  SplitArgs sa = {n, 1, nullptr, nullptr, nwl};
  const int parts = split_parts32(n, p.Sk, BK, device_cus(), CAUSAL, p.Sq);
  if (parts >= 2) {
    // every block is split; one key range of all of them takes part_bytes
    const size_t part_bytes = (size_t)n * nwl * NQB * (NDB + 1) * 64 * sizeof(f32x4);
    f32x4* ws = nullptr;
    int* cnt = nullptr;
    const int fit = bind_exchange(p, parts, part_bytes, 2 * n * nwl, &ws, &cnt);
    if (fit >= 2) sa = SplitArgs{0, fit, ws, cnt, nwl};
  }
  if (p.dry) return hipSuccess;
  const int nwg = sa.nfull + (n - sa.nfull) * sa.nparts;
  hipLaunchKernelGGL((attn_fwd_mfma32<DK, NW, NQB, BK, CAUSAL, ELEM, MASK>), dim3(nwg), dim3(NW * 64), 0, stream,
                     p, sa);
  return hipGetLastError();
}

template <int DK, bool CAUSAL, bool ELEM, bool MASK>
hipError_t launch_mfma32_inst(const FwdParams& p, hipStream_t stream) {
  constexpr int BK = (DK <= 128) ? 32 : 16;
  if constexpr (!CAUSAL && DK <= 64) {
    const int n = p.B * p.H * ((p.Sq + 63) / 64);
    if (tile_keys32(DK, n, p.Sk, device_cus(), CAUSAL) == 64)
      return launch_mfma32_bk<DK, CAUSAL, ELEM, 64, MASK>(p, stream);
  }
  return launch_mfma32_bk<DK, CAUSAL, ELEM, BK, MASK>(p, stream);
}

static const int kMfma32Dk[] = {16, 32, 40, 48, 64, 80, 96, 128, 160, 192, 256};

int mfma32_bucket(int D) {
  for (int dk : kMfma32Dk)
    if (D <= dk) return dk;
  return -1;
}

template <bool CAUSAL, bool ELEM, bool MASK = false>
static hipError_t launch_mfma32_dk(const FwdParams& p, int dk, hipStream_t s) {
  switch (dk) {
    case 16: return launch_mfma32_inst<16, CAUSAL, ELEM, MASK>(p, s);
    case 32: return launch_mfma32_inst<32, CAUSAL, ELEM, MASK>(p, s);
    case 40: return launch_mfma32_inst<40, CAUSAL, ELEM, MASK>(p, s);
    case 48: return launch_mfma32_inst<48, CAUSAL, ELEM, MASK>(p, s);
    case 64: return launch_mfma32_inst<64, CAUSAL, ELEM, MASK>(p, s);
    case 80: return launch_mfma32_inst<80, CAUSAL, ELEM, MASK>(p, s);
    case 96: return launch_mfma32_inst<96, CAUSAL, ELEM, MASK>(p, s);
    case 128: return launch_mfma32_inst<128, CAUSAL, ELEM, MASK>(p, s);
    case 160: return launch_mfma32_inst<160, CAUSAL, ELEM, MASK>(p, s);
    case 192: return launch_mfma32_inst<192, CAUSAL, ELEM, MASK>(p, s);
    case 256: return launch_mfma32_inst<256, CAUSAL, ELEM, MASK>(p, s);
  }
  return hipErrorInvalidValue;
}

hipError_t launch_mfma32(const FwdParams& p, bool causal, hipStream_t s) {
  const int dk = mfma32_bucket(p.D);
  if (dk < 0) return hipErrorInvalidValue;
  if (p.mask_kind != MASK_NONE) {
    // masked calls arrive with whole, 16-byte aligned rows (the ABI checks)
    if (p.elem_rows) return hipErrorNotSupported;
    return causal ? launch_mfma32_dk<true, false, true>(p, dk, s) : launch_mfma32_dk<false, false, true>(p, dk, s);
  }
  if (p.elem_rows)
    return causal ? launch_mfma32_dk<true, true>(p, dk, s) : launch_mfma32_dk<false, true>(p, dk, s);
  return causal ? launch_mfma32_dk<true, false>(p, dk, s) : launch_mfma32_dk<false, false>(p, dk, s);
}

void describe_mfma32(int D, int B, int H, int Sq, int Sk, bool causal, char* buf, int len) {
  const int dk = mfma32_bucket(D);
  const int bq = 64;
  const int n = B * H * ((Sq + bq - 1) / bq), cus = device_cus();
  const int bk = tile_keys32(dk, n, Sk, cus, causal);
  const int parts = split_parts32(n, Sk, bk, cus, causal, Sq);
  char split[48] = "";
  if (parts >= 2) snprintf(split, sizeof split, " key-split: %d x %d parts", n, parts);
  snprintf(buf, len, "mfma32 16x16x4f32 S^T-form: DK=%d DPV=%d waves=4 BQ=%d BK=%d qblocks=%d%s%s", dk,
           (dk + 15) / 16 * 16, bq, bk, (Sq + bq - 1) / bq, split,
           D % 4 != 0 ? " narrow rows" : "");
}

}  // namespace cmpext3
