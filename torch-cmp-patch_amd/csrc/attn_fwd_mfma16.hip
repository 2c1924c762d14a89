// Fused attention forward for fp16 / bf16 on gfx950 MFMA (v_mfma_f32_32x32x16_{f16,bf16}).
//
// Work split: one workgroup = NW waves = one (batch, head) pair x BQ = 32*NW
// query rows; each wave owns 32 query rows for the whole key sweep.  K/V are
// streamed in tiles of BK keys through double-buffered LDS; the next tile's
// global loads are in flight while the current one is computed.
//
// Layout trick: the kernel computes S^T = K Q^T (rows = keys, columns =
// queries) instead of S = Q K^T.  In the 32x32 MFMA accumulator a lane holds
// one column, so every lane owns one query row: the running max, running sum
// and the rescale of the output are lane-local, and a row reduction costs one
// v_permlane32_swap between the two 16-key halves.  The output is accumulated
// transposed as well, O^T = V^T P^T, so P^T goes from the score accumulator
// straight into the B operand of the PV MFMA without touching LDS.  To make
// the eight keys a lane contributes to one PV k-slice contiguous, K rows are
// fed to the score MFMA in a bit-permuted order (bits 2 and 3 of the row index
// swapped), which leaves every lane holding keys 16c+8h .. 16c+8h+7 of chunk c.
// V is staged in LDS transposed (V^T, keys contiguous) so that each PV A
// operand is a single 16-byte LDS read.
//
// Reference algorithm: src/cuda/fp16_flash_attention_hfma2.cu:72-243 (online
// exp2 softmax in fp32 with fp32 output accumulator and one final 1/l).  The
// reference's bf16 path casts to fp16 at the boundary (src/main.cpp:1623-1627);
// here bf16 runs natively on the bf16 MFMA.
#include "attn_common.h"

namespace cmpext3 {

template <typename T> struct Elt;

template <> struct Elt<_Float16> {
  static __device__ __forceinline__ f32x16 mma(u32x4 a, u32x4 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a),
                                                  __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
  }
  static __device__ __forceinline__ uint32_t pack(float a, float b) {
    const _Float16 x = (_Float16)a, y = (_Float16)b;
    return (uint32_t)__builtin_bit_cast(uint16_t, x) |
           ((uint32_t)__builtin_bit_cast(uint16_t, y) << 16);
  }
};

template <> struct Elt<__bf16> {
  static __device__ __forceinline__ f32x16 mma(u32x4 a, u32x4 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a),
                                                   __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
  }
  static __device__ __forceinline__ uint32_t pack(float a, float b) {
    const __bf16 x = (__bf16)a, y = (__bf16)b;
    return (uint32_t)__builtin_bit_cast(uint16_t, x) |
           ((uint32_t)__builtin_bit_cast(uint16_t, y) << 16);
  }
};

// MFMA row m of a 32-key block reads K row perm_row(m): bits 2 and 3 swapped.
__device__ __forceinline__ int perm_row(int m) {
  return (m & 0x13) | ((m & 4) << 1) | ((m & 8) >> 1);
}

// Key offset (inside a 32-key block) of accumulator element r in half hh,
// given the permuted K feed above: MFMA row 8*(r/4) + 4*hh + r%4.
__device__ __forceinline__ int acc_key(int r, int hh) {
  const int i = r >> 2, j = r & 3;
  return 16 * (i >> 1) + 8 * hh + 4 * (i & 1) + j;
}

// DK: head dim padded to a multiple of 16 (score k-steps); DP: padded to a
// multiple of 32 (output rows of the PV MFMA).  D <= DK is zero-filled.
template <typename T, int DK, int DP, int NW, int BK, bool CAUSAL>
__global__ void __launch_bounds__(NW * 64)
attn_fwd_mfma16(const FwdParams p) {
  constexpr int NT = NW * 64;
  constexpr int BQ = NW * 32;
  constexpr int RSK = DK + 8;       // K tile row stride in halves (16 B pad)
  constexpr int RSV = BK + 8;       // V^T tile row stride in halves
  constexpr int KTILE = BK * RSK;
  constexpr int VTILE = DP * RSV;
  constexpr int KCH = DK / 8;       // 16-byte chunks per K row
  constexpr int VCH = DP / 8;
  constexpr int KLD = (BK * KCH + NT - 1) / NT;
  constexpr int VLD = (BK * VCH + NT - 1) / NT;
  constexpr int NKB = BK / 32;      // 32-key blocks per tile
  constexpr int NCH = BK / 16;      // 16-key PV k-slices per tile
  constexpr int NDB = DP / 32;      // 32-row output blocks
  constexpr int NKS = DK / 16;      // score k-steps
  static_assert(BK % 32 == 0 && DK % 16 == 0 && DP % 32 == 0 && DK <= DP, "tile shape");

  __shared__ __attribute__((aligned(16))) uint16_t lds[2 * (KTILE + VTILE)];

  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  const int lane = tid & 63;
  const int l32 = lane & 31;
  const int hh = lane >> 5;

  // ---- which (batch, head, query block) this workgroup owns
  const int tile = xcd_remap(blockIdx.x, p.n_wg);
  const int bh = tile / p.n_qblk;
  int qblk = tile - bh * p.n_qblk;
  if (CAUSAL) qblk = p.n_qblk - 1 - qblk;  // longest key sweeps first
  const int b = bh / p.H;
  const int h = bh - b * p.H;
  const int q0 = qblk * BQ;

  const uint16_t* __restrict__ qg = (const uint16_t*)p.q + b * p.q_b + h * p.q_h;
  const uint16_t* __restrict__ kg = (const uint16_t*)p.k + b * p.k_b + h * p.k_h;
  const uint16_t* __restrict__ vg = (const uint16_t*)p.v + b * p.v_b + h * p.v_h;
  uint16_t* __restrict__ og = (uint16_t*)p.o + b * p.o_b + h * p.o_h;

  const int Sq = p.Sq, Sk = p.Sk, D = p.D;
  const int qw0 = q0 + wave * 32;      // first query row of this wave
  const int qrow = qw0 + l32;          // the query row this lane owns

  // ---- key range of this workgroup
  int kend = Sk;
  if (CAUSAL) kend = min(Sk, q0 + BQ);
  const int ntiles = (kend + BK - 1) / BK;

  // ---- Q as the B operand of S^T = K Q^T: lane holds Q[qrow][16s + 8hh .. +8]
  u32x4 qf[NKS];
#pragma unroll
  for (int s = 0; s < NKS; ++s) {
    const int d = 16 * s + 8 * hh;
    u32x4 x = {0u, 0u, 0u, 0u};
    if (qrow < Sq && d < D) x = *(const u32x4*)(qg + (int64_t)qrow * p.q_s + d);
    x ^= p.q_sign;
    qf[s] = x;
  }

  f32x16 oacc[NDB];
#pragma unroll
  for (int db = 0; db < NDB; ++db) oacc[db] = (f32x16){};
  float m_run = -INFINITY;
  float l_run = 0.f;
  const float c = p.c;

  // ---- global -> register staging of one K/V tile
  u32x4 kreg[KLD], vreg[VLD];
  auto load_tile = [&](int t) {
    const int k0 = t * BK;
#pragma unroll
    for (int it = 0; it < KLD; ++it) {
      const int ci = it * NT + tid;
      const int r = ci / KCH, c8 = ci - (ci / KCH) * KCH;
      u32x4 x = {0u, 0u, 0u, 0u};
      if ((BK * KCH % NT == 0 || ci < BK * KCH) && k0 + r < Sk && 8 * c8 < D)
        x = *(const u32x4*)(kg + (int64_t)(k0 + r) * p.k_s + 8 * c8);
      kreg[it] = x;
    }
#pragma unroll
    for (int it = 0; it < VLD; ++it) {
      const int ci = it * NT + tid;
      const int r = ci / VCH, c8 = ci - (ci / VCH) * VCH;
      u32x4 x = {0u, 0u, 0u, 0u};
      if ((BK * VCH % NT == 0 || ci < BK * VCH) && k0 + r < Sk && 8 * c8 < D)
        x = *(const u32x4*)(vg + (int64_t)(k0 + r) * p.v_s + 8 * c8);
      vreg[it] = x;
    }
  };
  auto store_tile = [&](int buf) {
    uint16_t* ks = lds + buf * (KTILE + VTILE);
    uint16_t* vt = ks + KTILE;
#pragma unroll
    for (int it = 0; it < KLD; ++it) {
      const int ci = it * NT + tid;
      if (BK * KCH % NT == 0 || ci < BK * KCH) {
        const int r = ci / KCH, c8 = ci - (ci / KCH) * KCH;
        *(u32x4*)(ks + r * RSK + 8 * c8) = kreg[it];
      }
    }
#pragma unroll
    for (int it = 0; it < VLD; ++it) {
      const int ci = it * NT + tid;
      if (BK * VCH % NT == 0 || ci < BK * VCH) {
        const int r = ci / VCH, c8 = ci - (ci / VCH) * VCH;
        const u32x4 x = vreg[it];
        uint16_t* dst = vt + (8 * c8) * RSV + r;
#pragma unroll
        for (int w = 0; w < 4; ++w) {
          dst[(2 * w) * RSV] = (uint16_t)(x[w] & 0xffffu);
          dst[(2 * w + 1) * RSV] = (uint16_t)(x[w] >> 16);
        }
      }
    }
  };

  if (ntiles > 0) load_tile(0);

  for (int t = 0; t < ntiles; ++t) {
    const int buf = t & 1;
    store_tile(buf);
    __syncthreads();
    if (t + 1 < ntiles) load_tile(t + 1);

    const int k0 = t * BK;
    // keys of this tile visible to some row of this wave?
    const bool active = !CAUSAL || k0 <= qw0 + 31;
    if (active) {
      const uint16_t* ks = lds + buf * (KTILE + VTILE);
      const uint16_t* vt = ks + KTILE;

      // ---- S^T blocks (32 keys x 32 queries each)
      f32x16 sacc[NKB];
#pragma unroll
      for (int kb = 0; kb < NKB; ++kb) {
        f32x16 acc = {};
        const uint16_t* krow = ks + (32 * kb + perm_row(l32)) * RSK + 8 * hh;
#pragma unroll
        for (int s = 0; s < NKS; ++s) {
          const u32x4 a = *(const u32x4*)(krow + 16 * s);
          acc = Elt<T>::mma(a, qf[s], acc);
        }
        sacc[kb] = acc;
      }

      // ---- masking (key tail, causal diagonal): masked tiles switch to the
      // pre-scaled domain so that -inf never meets a zero scale.
      const bool need_mask = (k0 + BK > Sk) || (CAUSAL && k0 + BK - 1 > qw0);
      float cm = c;
      if (need_mask) {
#pragma unroll
        for (int kb = 0; kb < NKB; ++kb) {
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const int key = k0 + 32 * kb + acc_key(r, hh);
            const bool dead = key >= Sk || (CAUSAL && key > qrow);
            sacc[kb][r] = dead ? -INFINITY : sacc[kb][r] * c;
          }
        }
        cm = 1.f;
      }

      // ---- online softmax (exp2 domain), lane-local per query row
      float mx = -INFINITY;
#pragma unroll
      for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
        for (int r = 0; r < 16; ++r) mx = fmaxf(mx, sacc[kb][r]);
      mx = xhalf_max(mx);
      const float m_tile = (mx == -INFINITY) ? -INFINITY : mx * cm;
      const float m_new = fmaxf(m_run, m_tile);
      const float m_use = (m_new == -INFINITY) ? 0.f : m_new;
      const float alpha = fast_exp2(m_run - m_use);
      m_run = m_new;
      l_run *= alpha;
#pragma unroll
      for (int db = 0; db < NDB; ++db) oacc[db] *= alpha;

      u32x4 pf[NCH];
#pragma unroll
      for (int kb = 0; kb < NKB; ++kb) {
#pragma unroll
        for (int cc = 0; cc < 2; ++cc) {
          u32x4 w;
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const float p0 = fast_exp2(sacc[kb][8 * cc + 2 * e] * cm - m_use);
            const float p1 = fast_exp2(sacc[kb][8 * cc + 2 * e + 1] * cm - m_use);
            l_run += p0 + p1;
            w[e] = Elt<T>::pack(p0, p1);
          }
          pf[2 * kb + cc] = w;
        }
      }

      // ---- O^T += V^T P^T
#pragma unroll
      for (int db = 0; db < NDB; ++db) {
        const uint16_t* vrow = vt + (32 * db + l32) * RSV + 8 * hh;
#pragma unroll
        for (int ch = 0; ch < NCH; ++ch) {
          const u32x4 a = *(const u32x4*)(vrow + 16 * ch);
          oacc[db] = Elt<T>::mma(a, pf[ch], oacc[db]);
        }
      }
    }
  }

  // ---- epilogue: combine the two halves' partial sums, normalise, store
  const float l_tot = xhalf_sum(l_run);
  const float inv = 1.f / l_tot;
  if (qrow < Sq) {
    uint16_t* orow = og + (int64_t)qrow * p.o_s;
#pragma unroll
    for (int db = 0; db < NDB; ++db) {
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
}

// ---------------------------------------------------------------------------
// host-side launchers (one per compiled instance)
// ---------------------------------------------------------------------------

template <typename T, int DK, bool CAUSAL>
hipError_t launch_mfma16_inst(const FwdParams& p0, hipStream_t stream) {
  constexpr int DP = (DK + 31) / 32 * 32;
  constexpr int NW = 4;
  constexpr int BK = (DK <= 128) ? 64 : 32;
  FwdParams p = p0;
  p.n_qblk = (p.Sq + NW * 32 - 1) / (NW * 32);
  p.n_wg = p.B * p.H * p.n_qblk;
  if (p.n_wg == 0) return hipSuccess;
  hipLaunchKernelGGL((attn_fwd_mfma16<T, DK, DP, NW, BK, CAUSAL>), dim3(p.n_wg), dim3(NW * 64), 0,
                     stream, p);
  return hipGetLastError();
}

// Head-dim buckets; D is zero-padded up to the bucket inside the kernel.
static const int kMfma16Dk[] = {32, 48, 64, 80, 96, 128, 160, 192, 256};

int mfma16_bucket(int D) {
  for (int dk : kMfma16Dk)
    if (D <= dk) return dk;
  return -1;
}

template <typename T, bool CAUSAL>
static hipError_t launch_mfma16_dk(const FwdParams& p, int dk, hipStream_t s) {
  switch (dk) {
    case 32: return launch_mfma16_inst<T, 32, CAUSAL>(p, s);
    case 48: return launch_mfma16_inst<T, 48, CAUSAL>(p, s);
    case 64: return launch_mfma16_inst<T, 64, CAUSAL>(p, s);
    case 80: return launch_mfma16_inst<T, 80, CAUSAL>(p, s);
    case 96: return launch_mfma16_inst<T, 96, CAUSAL>(p, s);
    case 128: return launch_mfma16_inst<T, 128, CAUSAL>(p, s);
    case 160: return launch_mfma16_inst<T, 160, CAUSAL>(p, s);
    case 192: return launch_mfma16_inst<T, 192, CAUSAL>(p, s);
    case 256: return launch_mfma16_inst<T, 256, CAUSAL>(p, s);
  }
  return hipErrorInvalidValue;
}

hipError_t launch_mfma16(const FwdParams& p, bool bf16, bool causal, hipStream_t s) {
  const int dk = mfma16_bucket(p.D);
  if (dk < 0) return hipErrorInvalidValue;
  if (bf16) return causal ? launch_mfma16_dk<__bf16, true>(p, dk, s) : launch_mfma16_dk<__bf16, false>(p, dk, s);
  return causal ? launch_mfma16_dk<_Float16, true>(p, dk, s) : launch_mfma16_dk<_Float16, false>(p, dk, s);
}

void describe_mfma16(int D, int Sq, char* buf, int len) {
  const int dk = mfma16_bucket(D);
  snprintf(buf, len, "mfma16 32x32x16 S^T-form: DK=%d DP=%d waves=4 BQ=128 BK=%d qblocks=%d", dk,
           (dk + 31) / 32 * 32, dk <= 128 ? 64 : 32, (Sq + 127) / 128);
}

}  // namespace cmpext3
