// Fused attention forward for fp16 / bf16 on gfx950 MFMA (v_mfma_f32_32x32x16_{f16,bf16}).
// Kernel template; attn_fwd_mfma16.hip instantiates the shipped tile table.
//
// Work split: a workgroup owns one (batch, head) pair and BQ = NW * QB * 32
// query rows; each of its NW waves owns QB blocks of 32 query rows for the
// whole key sweep.  K/V are streamed in tiles of BK keys through
// double-buffered LDS, and the next tile's global loads are in flight while
// the current one is computed.
//
// S^T form.  The kernel computes S^T = K Q^T (rows = keys, columns = queries).
// In the 32x32 MFMA accumulator a lane holds one column, so each lane owns one
// query row: its running max, running sum and output rescale are lane-local,
// and a row reduction is one v_permlane32_swap between the two 16-key halves.
// The output is accumulated transposed too, O^T = V^T P^T, so P^T goes from
// the score accumulator straight into the B operand of the PV MFMA.  K rows
// are fed to the score MFMA in a bit-permuted order (bits 2 and 3 of the row
// index swapped) so that each lane ends up holding 8 consecutive keys per
// 16-key PV slice.  V stays row-major in LDS; its A operand (8 keys at one d
// per lane) is read with ds_read_b64_tr_b16, whose 16-lane transpose turns
// four rows of 16 d's into 4 consecutive keys per lane.
//
// VALU diet (at D = 64 the softmax costs as much issue time as the MFMAs):
//  * PRESCALE: Q is multiplied by scale*log2(e) once at load, and the score
//    MFMA chain starts from a "bias" accumulator holding -m (the row's
//    current exp2 offset), so the accumulator already holds s*c - m and
//    p = exp2(acc) needs no per-score FMA.  Used for fp16 when |c| <= 1, so
//    the scaled Q cannot overflow.  Otherwise scores are scaled per element.
//  * Lazy rescale: the offset m is only raised when a tile's row maximum
//    exceeds it by more than 8 (log2 units); then P <= 2^8, which fp16/bf16
//    and the fp32 sums hold exactly enough.  The rescale of O and l is a
//    wave-uniform branch that is almost never taken after the first tile.
//  * P is packed with v_cvt_pk_{f16,bf16}_f32 and summed with v_dot2 into an
//    fp32 row sum, so the normaliser uses exactly the rounded P that the PV
//    MFMA consumes.
//
// Key split (non-causal launches with fewer query blocks than CUs: decode
// steps and short query sweeps, above all at head dims over 128 where one
// workgroup fills a CU): each block's key range is cut into parts run by
// separate workgroups; every part leaves its fp32 (O, m, l) in the exchange
// buffer and the last part of a (block, wave) to finish merges all of them in
// part order (its own from registers) and writes the output, as in
// attn_fwd_mfma32.hip.  Grouped-query launches with few query rows arrive
// with the query heads of a K/V head packed into the rows of one problem
// (FwdParams::pack_sq), so that K/V is streamed once per K/V head.
//
// Reference algorithm: src/cuda/fp16_flash_attention_hfma2.cu:72-243 (Q
// pre-scaled by scale*log2e, exp2 online softmax with fp32 running max/sum and
// fp32 output accumulator, one final 1/l).  The reference's bf16 path casts to
// fp16 at the boundary (src/main.cpp:1623-1627); here bf16 runs natively.
#pragma once

#include "attn_common.h"

namespace cmpext3 {

typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef short i16x4 __attribute__((ext_vector_type(4)));

template <typename T> struct Elt;

template <> struct Elt<_Float16> {
  static __device__ __forceinline__ f32x16 mma(u32x4 a, u32x4 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a),
                                                  __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
  }
  static __device__ __forceinline__ uint32_t pack(float a, float b) {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2){a, b}, f16x2));
  }
  static __device__ __forceinline__ f32x2 unpack(uint32_t w) {
    return __builtin_convertvector(__builtin_bit_cast(f16x2, w), f32x2);
  }
  // acc + lo(w) + hi(w) in fp32
  static __device__ __forceinline__ float sum2(uint32_t w, float acc) {
    return __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2, w), (f16x2){1.0f16, 1.0f16}, acc, false);
  }
};

template <> struct Elt<__bf16> {
  static __device__ __forceinline__ f32x16 mma(u32x4 a, u32x4 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a),
                                                   __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
  }
  static __device__ __forceinline__ uint32_t pack(float a, float b) {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2){a, b}, bf16x2));
  }
  static __device__ __forceinline__ f32x2 unpack(uint32_t w) {
    return (f32x2){__uint_as_float(w << 16), __uint_as_float(w & 0xffff0000u)};
  }
  static __device__ __forceinline__ float sum2(uint32_t w, float acc) {
    const bf16x2 one = {(__bf16)1.0f, (__bf16)1.0f};
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, w), one, acc, false);
  }
};

// MFMA row m of a 32-key block reads K row perm_row(m): bits 2 and 3 swapped.
__device__ __forceinline__ int perm_row(int m) {
  return (m & 0x13) | ((m & 4) << 1) | ((m & 8) >> 1);
}

// Key (inside its 32-key block) of accumulator element r of half hh, given the
// permuted K feed: MFMA row 8*(r/4) + 4*hh + r%4 -> key 16*(r/8) + 8*hh + r%8.
__device__ __forceinline__ int acc_key(int r, int hh) {
  return 16 * (r >> 3) + 8 * hh + (r & 7);
}

__device__ __forceinline__ uint2 lds_tr16_b64(const uint16_t* p) {
  typedef __attribute__((address_space(3))) i16x4 lds_i16x4;
  const i16x4 v = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(p));
  return __builtin_bit_cast(uint2, v);
}

// Attention mask (FwdParams::mask) of 8 consecutive keys of one query row,
// applied to the exp2-domain scores sc[r0 .. r0 + 7]: a zero bool removes
// the key (-inf), float kinds are added times log2(e).  `off` is the byte
// offset of the first key in the mask buffer (reads past its end return
// zero).  One 8-, 16- or 32-byte read, or (narrow) one read per element.
__device__ __forceinline__ void mask_run8(f32x16& sc, int r0, const __amdgpu_buffer_rsrc_t& mrs, int off,
                                          int kind, bool narrow) {
  if (narrow) {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      if (kind == MASK_BOOL) {
        if (__builtin_amdgcn_raw_buffer_load_b8(mrs, off + i, 0, 0) == 0) sc[r0 + i] = -INFINITY;
      } else if (kind == MASK_F32) {
        const float a = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(mrs, off + 4 * i, 0, 0));
        sc[r0 + i] = __builtin_fmaf(a, kLog2e, sc[r0 + i]);
      } else {
        const uint32_t hb = __builtin_amdgcn_raw_buffer_load_b16(mrs, off + 2 * i, 0, 0);
        const float a = kind == MASK_F16 ? (float)__builtin_bit_cast(_Float16, (uint16_t)hb) : __uint_as_float(hb << 16);
        sc[r0 + i] = __builtin_fmaf(a, kLog2e, sc[r0 + i]);
      }
    }
    return;
  }
  if (kind == MASK_BOOL) {
    const u32x2 w = __builtin_bit_cast(u32x2, __builtin_amdgcn_raw_buffer_load_b64(mrs, off, 0, 0));
#pragma unroll
    for (int i = 0; i < 8; ++i)
      if (((w[i >> 2] >> (8 * (i & 3))) & 0xffu) == 0u) sc[r0 + i] = -INFINITY;
  } else if (kind == MASK_F32) {
#pragma unroll
    for (int hv = 0; hv < 2; ++hv) {
      const f32x4 a = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(mrs, off + 16 * hv, 0, 0));
#pragma unroll
      for (int i = 0; i < 4; ++i) sc[r0 + 4 * hv + i] = __builtin_fmaf(a[i], kLog2e, sc[r0 + 4 * hv + i]);
    }
  } else {
    const u32x4 w = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(mrs, off, 0, 0));
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const f32x2 a = kind == MASK_F16 ? Elt<_Float16>::unpack(w[i]) : Elt<__bf16>::unpack(w[i]);
      sc[r0 + 2 * i] = __builtin_fmaf(a[0], kLog2e, sc[r0 + 2 * i]);
      sc[r0 + 2 * i + 1] = __builtin_fmaf(a[1], kLog2e, sc[r0 + 2 * i + 1]);
    }
  }
}

// The mask words of one run of 8 keys (whole runs: an 8-, 16- or 32-byte
// read), split from their use so that a tile can test them first.
struct MaskRun8 {
  u32x4 w0, w1;  // bool: w0.xy; f16/bf16: w0; f32: w0, w1
};
__device__ __forceinline__ MaskRun8 mask_load8(const __amdgpu_buffer_rsrc_t& mrs, int off, int kind) {
  MaskRun8 m;
  m.w1 = (u32x4){0u, 0u, 0u, 0u};
  if (kind == MASK_BOOL) {
    const u32x2 w = __builtin_bit_cast(u32x2, __builtin_amdgcn_raw_buffer_load_b64(mrs, off, 0, 0));
    m.w0 = (u32x4){w[0], w[1], 0x01010101u, 0x01010101u};
  } else {
    m.w0 = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(mrs, off, 0, 0));
    if (kind == MASK_F32) m.w1 = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(mrs, off + 16, 0, 0));
  }
  return m;
}
// True when the run leaves every score as it is: no zero bool byte, or every
// additive value +0 (bit pattern zero).
__device__ __forceinline__ bool mask_run_keeps(const MaskRun8& m, int kind) {
  if (kind == MASK_BOOL) {
    uint32_t z = 0;  // high bit of every zero byte (the classic has-zero-byte test)
#pragma unroll
    for (int i = 0; i < 2; ++i) z |= (m.w0[i] - 0x01010101u) & ~m.w0[i] & 0x80808080u;
    return z == 0u;
  }
  const u32x4 o = m.w0 | m.w1;
  return (o[0] | o[1] | o[2] | o[3]) == 0u;
}
// Apply a loaded run to sc[r0 .. r0 + 7] as mask_run8 does.
__device__ __forceinline__ void mask_apply8(f32x16& sc, int r0, const MaskRun8& m, int kind) {
  if (kind == MASK_BOOL) {
#pragma unroll
    for (int i = 0; i < 8; ++i)
      if (((m.w0[i >> 2] >> (8 * (i & 3))) & 0xffu) == 0u) sc[r0 + i] = -INFINITY;
  } else if (kind == MASK_F32) {
#pragma unroll
    for (int i = 0; i < 8; ++i)
      sc[r0 + i] = __builtin_fmaf(__uint_as_float(i < 4 ? m.w0[i] : m.w1[i - 4]), kLog2e, sc[r0 + i]);
  } else {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const f32x2 a = kind == MASK_F16 ? Elt<_Float16>::unpack(m.w0[i]) : Elt<__bf16>::unpack(m.w0[i]);
      sc[r0 + 2 * i] = __builtin_fmaf(a[0], kLog2e, sc[r0 + 2 * i]);
      sc[r0 + 2 * i + 1] = __builtin_fmaf(a[1], kLog2e, sc[r0 + 2 * i + 1]);
    }
  }
}

// Bytes of the mask buffer of one (batch, head) that a kernel may read: up
// to key Sk - 1 of the last row (narrow), or up to Sk rounded up to 8.
__device__ __forceinline__ int64_t mask_span(const FwdParams& p, int mes) {
  return ((int64_t)(p.Sq - 1) * p.m_q + (p.mask_narrow ? p.Sk : (p.Sk + 7) / 8 * 8)) * mes;
}

constexpr float kSumHi = 256.0f;         // tile row sum above this: offset must rise
constexpr float kSumLo = 1.0f / 256.0f;  // first tile row sum below this: offset too high

// Chunk swizzle of LDS row r (DK / 8 sixteen-byte chunks per row).  For the
// K fragment reads (16 lanes: rows 0..15 of a 32-row block, one chunk), the
// transposed V reads (32 lanes: 4 consecutive rows x 4 consecutive chunks)
// and the 16-byte tile writes, every 64-bank LDS cycle hits distinct banks.
template <int DK>
__device__ __forceinline__ int lds_swz(int r) {
  if constexpr (DK == 32) return (r >> 2) & 3;
  else if constexpr (DK == 64) return (((r >> 1) & 1) << 2) | ((r >> 2) & 3);
  else return ((r & 3) << 2) | ((r >> 2) & 3);  // DK == 128
}

// DK: head dim padded to a multiple of 16 (score k-steps); DP: padded to a
// multiple of 32 (output rows of the PV MFMA).  Columns D..DP-1 are zero.
// OCC: waves per SIMD the register allocation must allow (occupancy target).
// OPT bit 0: raise the wave's issue priority (s_setprio) while it issues MFMAs.
// OPT bit 1: unpadded XOR-swizzled LDS rows instead of 16-byte padding (only
// for DK == DP in {32, 64, 128}).  OPT bit 2: decide the rescale from the
// tile's row sum after the exponentials instead of from the row max before
// them (measured slower on MI355X: the PV MFMAs then wait for the whole sum).
// The padded, max-first form is the default.  OPT bit 6: narrow rows
// (ld_cols16 / st_cols16x4, FwdParams::elem_rows): any head dim and any
// 2-byte aligned rows, read and written in 2-, 4- or 8-byte pieces, columns
// past D never touched.  OPT bit 4: an attention mask (p.mask) on every
// tile's scores.  OPT bit 5: each row's natural-log log-sum-exp goes to
// p.lse (the training forward; such launches are never key-split).
template <typename T, int DK, int DP, int NW, int QB, int BK, int OCC, bool CAUSAL, bool PRESCALE,
          int OPT = 0>
__global__ void __launch_bounds__(NW * 64) __attribute__((amdgpu_waves_per_eu(OCC)))
attn_fwd_mfma16(const FwdParams p, const SplitArgs sa) {
  constexpr int NT = NW * 64;
  constexpr int QPW = 32 * QB;          // query rows per wave
  constexpr int BQ = NW * QPW;
  // LDS rows padded by 16 bytes (a 64-row K/V tile then reads without
  // measurable bank conflicts), or unpadded with XOR-swizzled 16-byte chunks.
  constexpr bool SWZ = (OPT & 2) && (DK == DP) && (DK == 32 || DK == 64 || DK == 128);
  constexpr bool ELEM = (OPT & 64) != 0;
  constexpr bool MASK = (OPT & 16) != 0;
  constexpr int RSK = SWZ ? DK : DK + 8;  // K tile row stride (halves)
  constexpr int RSV = SWZ ? DP : DP + 8;  // V tile row stride (halves)
  constexpr int KTILE = BK * RSK;
  constexpr int VTILE = BK * RSV;
  constexpr int KCH = DK / 8;           // 16-byte chunks per K row
  constexpr int VCH = DP / 8;
  constexpr int KLD = (BK * KCH + NT - 1) / NT;
  constexpr int VLD = (BK * VCH + NT - 1) / NT;
  constexpr int NKB = BK / 32;          // 32-key blocks per tile
  constexpr int NCH = BK / 16;          // 16-key PV slices per tile
  constexpr int NDB = DP / 32;          // 32-row output blocks
  constexpr int NKS = DK / 16;          // score k-steps
  static_assert(BK % 32 == 0 && DK % 16 == 0 && DP % 32 == 0 && DK <= DP, "tile shape");

  __shared__ __attribute__((aligned(16))) uint16_t lds[2 * (KTILE + VTILE)];

  const int tid = thread_x();
  const int wave = tid >> 6;
  const int lane = tid & 63;
  const int l32 = lane & 31;
  const int hh = lane >> 5;

  // ---- which (batch, head, query block) and which part of its keys this
  // workgroup owns
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

  const uint16_t* __restrict__ qg = (const uint16_t*)p.q + b * p.q_b + h * p.q_h;
  const uint16_t* kg = (const uint16_t*)p.k + b * p.k_b + (h / p.kv_group) * p.k_h;
  const uint16_t* vg = (const uint16_t*)p.v + b * p.v_b + (h / p.kv_group) * p.v_h;
  uint16_t* __restrict__ og = (uint16_t*)p.o + b * p.o_b + h * p.o_h;

  const int Sq = p.Sq, Sk = p.Sk, D = p.D;
  const int qw0 = q0 + wave * QPW;      // first query row of this wave
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
  // this workgroup's key tiles [tbase, tbase + ntiles)
  const int ntall = (kend + BK - 1) / BK;
  const int tbase = part * ntall / nparts;
  const int ntiles = (part + 1) * ntall / nparts - tbase;

  // ---- Q as the B operand of S^T = K Q^T: lane holds Q[row][16s + 8hh .. +8]
  const float cq = p.q_sign ? -p.c : p.c;  // signed scale*log2(e) for PRESCALE
  u32x4 qf[QB][NKS];
#pragma unroll
  for (int qb = 0; qb < QB; ++qb) {
    const int row = qw0 + 32 * qb + l32;
#pragma unroll
    for (int s = 0; s < NKS; ++s) {
      const int d = 16 * s + 8 * hh;
      u32x4 x = {0u, 0u, 0u, 0u};
      if (row < Sq && d < D) {
        const uint16_t* src = qg + row_off(row, p.q_g, p.q_s) + d;
        x = ELEM ? ld_cols16(src, D - d, p.elem_rows) : *(const u32x4*)src;
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
      qf[qb][s] = x;
    }
  }

  // ---- running state per query block (lane = one query row)
  f32x16 oacc[QB][NDB];
  f32x16 bias[QB];
  float mb[QB], lsum[QB];
  bool first[QB];
#pragma unroll
  for (int qb = 0; qb < QB; ++qb) {
#pragma unroll
    for (int db = 0; db < NDB; ++db) oacc[qb][db] = (f32x16){};
    bias[qb] = (f32x16){};
    mb[qb] = 0.f;
    lsum[qb] = 0.f;
    first[qb] = true;
  }
  const float c = p.c;

  // ---- per-thread global/LDS offsets of its tile chunks (fixed across tiles)
  int kgo[KLD], klo[KLD], krow[KLD], kn[KLD];
  bool kok[KLD];
#pragma unroll
  for (int it = 0; it < KLD; ++it) {
    const int ci = it * NT + tid;
    const int r = ci / KCH, c8 = ci - r * KCH;
    krow[it] = r;
    kn[it] = D - 8 * c8;  // columns of the chunk inside the head dim (ELEM)
    kok[it] = (BK * KCH % NT == 0 || ci < BK * KCH) && 8 * c8 < D;
    kgo[it] = r * (int)p.k_s + 8 * c8;
    klo[it] = r * RSK + 8 * (SWZ ? (c8 ^ lds_swz<DK>(r)) : c8);
  }
  int vgo[VLD], vlo[VLD], vrow[VLD], vn[VLD];
  bool vok[VLD];
#pragma unroll
  for (int it = 0; it < VLD; ++it) {
    const int ci = it * NT + tid;
    const int r = ci / VCH, c8 = ci - r * VCH;
    vrow[it] = r;
    vn[it] = D - 8 * c8;
    vok[it] = (BK * VCH % NT == 0 || ci < BK * VCH) && 8 * c8 < D;
    vgo[it] = r * (int)p.v_s + 8 * c8;
    vlo[it] = r * RSV + 8 * (SWZ ? (c8 ^ lds_swz<DP>(r)) : c8);
  }
  const int64_t kstep = (int64_t)BK * p.k_s, vstep = (int64_t)BK * p.v_s;

  u32x4 kreg[KLD], vreg[VLD];
  // no zero-filled head-dim columns (element-granular rows always take the
  // checked path below)
  const bool cols_full = !ELEM && (D == DK) && (D == DP);
  auto load_tile = [&](int t) {
    const int k0 = (tbase + t) * BK;
    const uint16_t* kt = kg + (tbase + t) * kstep;
    const uint16_t* vt = vg + (tbase + t) * vstep;
    if (cols_full && k0 + BK <= Sk) {
      // interior tile: every chunk this thread owns is in bounds
#pragma unroll
      for (int it = 0; it < KLD; ++it)
        if (BK * KCH % NT == 0 || it * NT + tid < BK * KCH) kreg[it] = *(const u32x4*)(kt + kgo[it]);
#pragma unroll
      for (int it = 0; it < VLD; ++it)
        if (BK * VCH % NT == 0 || it * NT + tid < BK * VCH) vreg[it] = *(const u32x4*)(vt + vgo[it]);
      return;
    }
#pragma unroll
    for (int it = 0; it < KLD; ++it) {
      u32x4 x = {0u, 0u, 0u, 0u};
      if (kok[it] && k0 + krow[it] < Sk)
        x = ELEM ? ld_cols16(kt + kgo[it], kn[it], p.elem_rows) : *(const u32x4*)(kt + kgo[it]);
      kreg[it] = x;
    }
#pragma unroll
    for (int it = 0; it < VLD; ++it) {
      u32x4 x = {0u, 0u, 0u, 0u};
      if (vok[it] && k0 + vrow[it] < Sk)
        x = ELEM ? ld_cols16(vt + vgo[it], vn[it], p.elem_rows) : *(const u32x4*)(vt + vgo[it]);
      vreg[it] = x;
    }
  };
  auto store_tile = [&](int buf) {
    uint16_t* ks = lds + buf * (KTILE + VTILE);
    uint16_t* vs = ks + KTILE;
#pragma unroll
    for (int it = 0; it < KLD; ++it)
      if (BK * KCH % NT == 0 || it * NT + tid < BK * KCH) *(u32x4*)(ks + klo[it]) = kreg[it];
#pragma unroll
    for (int it = 0; it < VLD; ++it)
      if (BK * VCH % NT == 0 || it * NT + tid < BK * VCH) *(u32x4*)(vs + vlo[it]) = vreg[it];
  };

  // lane-constant parts of the LDS read addresses (halves within a tile)
  int k_rd[NKS];  // + 32*kb*RSK
  {
    const int r = perm_row(l32);
#pragma unroll
    for (int s = 0; s < NKS; ++s)
      k_rd[s] = r * RSK + (SWZ ? 8 * ((2 * s + hh) ^ lds_swz<DK>(r)) : 16 * s + 8 * hh);
  }
  const int jj = lane & 15, gg = lane >> 4;
  int v_rd[NDB][2];  // + 16*ch*RSV
#pragma unroll
  for (int db = 0; db < NDB; ++db)
#pragma unroll
    for (int half = 0; half < 2; ++half) {
      const int r = 8 * (gg >> 1) + (jj >> 2) + 4 * half;
      const int col = 32 * db + 16 * (gg & 1) + 4 * (jj & 3);
      v_rd[db][half] = r * RSV + (SWZ ? 8 * ((col >> 3) ^ lds_swz<DP>(r)) + (col & 7) : col);
    }

  // attention mask (MASK): a lane's 16 keys per 32-key block are 2 runs of 8
  // consecutive keys (acc_key), one read each (mask_run8); rows past Sq read
  // the last row (their output is never stored); reads past the readable span
  // (mask_span) return zero and keys at or past Sk are masked afterwards
  const int mes = p.mask_kind == MASK_BOOL ? 1 : p.mask_kind == MASK_F32 ? 4 : 2;
  const __amdgpu_buffer_rsrc_t mrs =
      uniform_rsrc(MASK ? (const void*)((const char*)p.mask + (b * p.m_b + h * p.m_h) * mes) : p.q,
                   MASK ? mask_span(p, mes) : 0);
  int mrow_off[QB];
#pragma unroll
  for (int qb = 0; qb < QB; ++qb)
    mrow_off[qb] = MASK ? (int)((int64_t)min(qw0 + 32 * qb + l32, Sq - 1) * p.m_q * mes) : 0;

  if (ntiles > 0) load_tile(0);

  for (int t = 0; t < ntiles; ++t) {
    const int buf = t & 1;
    store_tile(buf);
    __syncthreads();
    if (t + 1 < ntiles) load_tile(t + 1);

    const int k0 = (tbase + t) * BK;
    const uint16_t* ks = lds + buf * (KTILE + VTILE);
    const uint16_t* vs = ks + KTILE;

#pragma unroll
    for (int qb = 0; qb < QB; ++qb) {
      const int qlo = qw0 + 32 * qb;      // first row of this query block
      if (CAUSAL && k0 > qlo + 31) continue;  // every key of the tile is in the future

      // ---- S^T blocks in the exp2 domain: x = s*c - m (PRESCALE: the MFMA
      // chain starts from bias = -m and Q already carries c)
      f32x16 sacc[NKB];
      const int qrow = qlo + l32;
      const bool need_mask = (k0 + BK > Sk) || (CAUSAL && k0 + BK - 1 > qlo);
      auto scores = [&]() {
#pragma unroll
        for (int kb = 0; kb < NKB; ++kb) {
          f32x16 acc = PRESCALE ? bias[qb] : (f32x16){};
          const uint16_t* kr = ks + 32 * kb * RSK;
          if (OPT & 1) __builtin_amdgcn_s_setprio(1);
#pragma unroll
          for (int s = 0; s < NKS; ++s) acc = Elt<T>::mma(*(const u32x4*)(kr + k_rd[s]), qf[qb][s], acc);
          if (OPT & 1) __builtin_amdgcn_s_setprio(0);
          sacc[kb] = acc;
        }
        if (!PRESCALE) {
#pragma unroll
          for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
            for (int r = 0; r < 16; ++r) sacc[kb][r] = __builtin_fmaf(sacc[kb][r], c, -mb[qb]);
        }
        if (MASK) {
#pragma unroll
          for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
            for (int run = 0; run < 2; ++run)
              mask_run8(sacc[kb], 8 * run, mrs, mrow_off[qb] + (k0 + 32 * kb + 16 * run + 8 * hh) * mes,
                        p.mask_kind, p.mask_narrow);
        }
        if (need_mask) {
#pragma unroll
          for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
              const int key = k0 + 32 * kb + acc_key(r, hh);
              if (key >= Sk || (CAUSAL && key > qrow)) sacc[kb][r] = -INFINITY;
            }
        }
      };
      scores();

      // ---- P = exp2(x) packed to T against the current offset; the tile's
      // row sum (this lane's half) from the packed values
      u32x4 pf[NCH];
      float ls[2];
      auto exp_pack = [&]() {
        ls[0] = 0.f;
        ls[1] = 0.f;  // two independent dot2 chains
#pragma unroll
        for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
          for (int cc = 0; cc < 2; ++cc) {
            u32x4 w;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              w[e] = Elt<T>::pack(fast_exp2(sacc[kb][8 * cc + 2 * e]),
                                  fast_exp2(sacc[kb][8 * cc + 2 * e + 1]));
              ls[e & 1] = Elt<T>::sum2(w[e], ls[e & 1]);
            }
            pf[2 * kb + cc] = w;
          }
      };
      // Raise the offset to the tile's row max (never lower it after the first
      // live tile); rescale O and l by 2^-delta.  Returns delta.
      auto rescale_to_max = [&]() {
        float mq = -INFINITY;
#pragma unroll
        for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
          for (int r = 0; r < 16; ++r) mq = fmaxf(mq, sacc[kb][r]);
        const float mx = xhalf_max(mq);
        float delta = first[qb] ? mx : fmaxf(mx, 0.f);
        if (mx == -INFINITY) delta = 0.f;
        const float alpha = fast_exp2(-delta);
        mb[qb] += delta;
        lsum[qb] *= alpha;
#pragma unroll
        for (int db = 0; db < NDB; ++db) oacc[qb][db] *= alpha;
        if (PRESCALE) bias[qb] = (f32x16){} - mb[qb];
        first[qb] = first[qb] && (mx == -INFINITY);
        return delta;
      };

      float lt;
      if (!(OPT & 4)) {
        // max-first: rescale when the tile max exceeds the offset by 8
        float mq = -INFINITY;
#pragma unroll
        for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
          for (int r = 0; r < 16; ++r) mq = fmaxf(mq, sacc[kb][r]);
        const bool need = xhalf_max(mq) > (first[qb] ? -INFINITY : 8.f);
        if (__builtin_amdgcn_ballot_w64(need)) {
          const float delta = rescale_to_max();
#pragma unroll
          for (int kb = 0; kb < NKB; ++kb) sacc[kb] -= delta;
        }
        exp_pack();
        lt = ls[0] + ls[1];
      } else {
        // ---- lazy rescale, decided from the tile sum: above 2^8 a P may
        // have left the headroom; on the first tile, below 2^-8 the offset
        // sits far above the scores.  Only then recompute the scores (the K
        // tile is still in LDS), take the row max and redo the exponentials;
        // the common path keeps no scores alive past the exponentials.
        exp_pack();
        lt = ls[0] + ls[1];
        const bool need = !(lt <= kSumHi) || (first[qb] && lt < kSumLo);
        if (__builtin_amdgcn_ballot_w64(need)) {
          // the clobber makes the K fragments be read again instead of the
          // first pass's scores being kept live for this branch
          asm volatile("" ::: "memory");
          scores();
          const float delta = rescale_to_max();
#pragma unroll
          for (int kb = 0; kb < NKB; ++kb) sacc[kb] -= delta;
          exp_pack();
          lt = ls[0] + ls[1];
        } else {
          first[qb] = false;
        }
      }
      lsum[qb] += lt;

      // ---- O^T += V^T P^T  (V^T fragments via the LDS transpose read)
      if (OPT & 1) __builtin_amdgcn_s_setprio(1);
#pragma unroll
      for (int db = 0; db < NDB; ++db) {
#pragma unroll
        for (int ch = 0; ch < NCH; ++ch) {
          const uint16_t* vp = vs + 16 * ch * RSV;
          const uint2 lo = lds_tr16_b64(vp + v_rd[db][0]);
          const uint2 hi = lds_tr16_b64(vp + v_rd[db][1]);
          const u32x4 a = {lo.x, lo.y, hi.x, hi.y};
          oacc[qb][db] = Elt<T>::mma(a, pf[ch], oacc[qb][db]);
        }
      }
      if (OPT & 1) __builtin_amdgcn_s_setprio(0);
    }
  }

  // ---- epilogue: combine the two halves' partial sums
  float lrow[QB];
#pragma unroll
  for (int qb = 0; qb < QB; ++qb) lrow[qb] = xhalf_sum(lsum[qb]);
  if (nparts > 1) {
    // Every part leaves its state and counts itself in; the last one in
    // merges and writes the output.  Device-scope (aux 16 = sc1) 16-byte
    // accesses, coherent across the XCDs' L2s.
    constexpr int NVB = 4 * NDB + 1;  // float4 vectors per query block: O, then (m, l)
    constexpr int NV = QB * NVB;
    const int sb = lb - sa.nfull, nwl = sa.nwl;
    const __amdgpu_buffer_rsrc_t wsr = uniform_rsrc(sa.ws, (int64_t)(sb + 1) * nparts * nwl * NV * 64 * 16);
    // vector k of part q's state for the rows of wave w
    auto voffw = [&](int q, int w, int k) { return ((((sb * nparts + q) * nwl + w) * NV + k) * 64 + lane) * 16; };
    auto voff = [&](int q, int k) { return voffw(q, wave, k); };
    auto st_ws = [&](f32x4 x, int off) {
      __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, x), wsr, off, 0, 16);
    };
    auto ld_ws = [&](int off) { return __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(wsr, off, 0, 16)); };
    auto frag = [](const f32x16& a, int i) { return (f32x4){a[4 * i], a[4 * i + 1], a[4 * i + 2], a[4 * i + 3]}; };
    if (nwl < NW) {
      // Rows in fewer waves than the workgroup has (decode steps, packed
      // query groups): the last part's whole workgroup merges.  The waves
      // with rows leave their state, the block is counted in once, and each
      // of the NW waves then merges a share of the (row wave, query block,
      // 32-column block) units of every part, all read from the exchange, so
      // the result is the same whichever part is last.  Nobody waits for
      // another workgroup.  (One wave merging a 256-wide output alone held
      // its accumulators and one part's loads at a time.)
      if (wave < nwl) {
#pragma unroll
        for (int qb = 0; qb < QB; ++qb) {
#pragma unroll
          for (int db = 0; db < NDB; ++db)
#pragma unroll
            for (int i = 0; i < 4; ++i) st_ws(frag(oacc[qb][db], i), voff(part, qb * NVB + 4 * db + i));
          st_ws((f32x4){lrow[qb] > 0.f ? mb[qb] : -INFINITY, lrow[qb], 0.f, 0.f}, voff(part, qb * NVB + 4 * NDB));
        }
      }
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
      lds_barrier();  // every wave's state is written and its LDS reads are done
      int* const flag = (int*)lds;
      if (tid == 0) {
        int* const ctr = sa.cnt + 2 * sb * nwl;
        const int old = __hip_atomic_fetch_add(ctr, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (old == nparts - 1) __hip_atomic_store(ctr, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        *flag = old == nparts - 1;
      }
      lds_barrier();
      if (__builtin_amdgcn_readfirstlane(*flag) == 0) return;
      asm volatile("" ::: "memory");  // the exchange loads stay after the count
      constexpr int CHM = 4;  // parts whose loads are in flight together
      for (int u = wave; u < nwl * QB * NDB; u += NW) {
        const int w2 = u / (QB * NDB), r = u - w2 * (QB * NDB), qb = r / NDB, db = r - qb * NDB;
        float mt = -INFINITY;
        for (int qa = 0; qa < nparts; qa += CHM) {
          float mq[CHM];
#pragma unroll
          for (int j = 0; j < CHM; ++j) mq[j] = ld_ws(voffw(min(qa + j, nparts - 1), w2, qb * NVB + 4 * NDB))[0];
#pragma unroll
          for (int j = 0; j < CHM; ++j) mt = fmaxf(mt, mq[j]);  // clamped repeats change nothing
        }
        f32x16 acc = (f32x16){};
        float l = 0.f;
        for (int qa = 0; qa < nparts; qa += CHM) {
          f32x4 ml[CHM], x[CHM][4];
#pragma unroll
          for (int j = 0; j < CHM; ++j) {
            const int qq = min(qa + j, nparts - 1);
            ml[j] = ld_ws(voffw(qq, w2, qb * NVB + 4 * NDB));
#pragma unroll
            for (int i = 0; i < 4; ++i) x[j][i] = ld_ws(voffw(qq, w2, qb * NVB + 4 * db + i));
          }
#pragma unroll
          for (int j = 0; j < CHM; ++j) {
            if (qa + j >= nparts) break;
            const float a = ml[j][0] == -INFINITY ? 0.f : fast_exp2(ml[j][0] - mt);
            l = __builtin_fmaf(ml[j][1], a, l);
#pragma unroll
            for (int i = 0; i < 16; ++i) acc[i] = __builtin_fmaf(x[j][i / 4][i % 4], a, acc[i]);
          }
        }
        const float inv = l > 0.f ? 1.f / l : 0.f;
        const int qrow = q0 + w2 * QPW + 32 * qb + l32;
        if (qrow < Sq) {
          uint16_t* orow = og + row_off(qrow, p.o_g, p.o_s);
#pragma unroll
          for (int g = 0; g < 4; ++g) {
            const int d = 32 * db + 8 * g + 4 * hh;
            if (d < D) {
              u32x2 w;
              w[0] = Elt<T>::pack(acc[4 * g + 0] * inv, acc[4 * g + 1] * inv);
              w[1] = Elt<T>::pack(acc[4 * g + 2] * inv, acc[4 * g + 3] * inv);
              if (ELEM)
                st_cols16x4(orow + d, w, D - d, p.elem_rows);
              else
                *(u32x2*)(orow + d) = w;
            }
          }
        }
      }
      return;
    }
    // a wave whose rows all lie past Sq has nothing to exchange; every part
    // of the block agrees on that
    if (qw0 >= Sq) return;
    int* const ctr = sa.cnt + 2 * (sb * nwl + wave);  // parts in (the second counter is unused here)
    // a row that holds nothing from this part's keys: offset -inf
    float m_own[QB];
#pragma unroll
    for (int qb = 0; qb < QB; ++qb) {
      m_own[qb] = lrow[qb] > 0.f ? mb[qb] : -INFINITY;
#pragma unroll
      for (int db = 0; db < NDB; ++db)
#pragma unroll
        for (int i = 0; i < 4; ++i) st_ws(frag(oacc[qb][db], i), voff(part, qb * NVB + 4 * db + i));
      st_ws((f32x4){m_own[qb], lrow[qb], 0.f, 0.f}, voff(part, qb * NVB + 4 * NDB));
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    int old = 0;
    if (lane == 0) old = __hip_atomic_fetch_add(ctr, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    old = __builtin_amdgcn_readfirstlane(old);
    if (old != nparts - 1) return;
    if (lane == 0) __hip_atomic_store(ctr, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    asm volatile("" ::: "memory");  // the exchange loads stay after the count
    // merge in part order, this part from its registers: the same
    // instructions on the same values whichever part arrives last.  CH parts'
    // loads are issued together (fewer memory round trips) where the
    // registers allow; part indices past the last are clamped and dropped.
    constexpr int CH = NDB <= 2 ? 2 : 1;
#pragma unroll
    for (int qb = 0; qb < QB; ++qb) {
      float mt = m_own[qb];
      for (int q0 = 0; q0 < nparts; q0 += 4) {
        float mq[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) mq[j] = ld_ws(voff(min(q0 + j, nparts - 1), qb * NVB + 4 * NDB))[0];
#pragma unroll
        for (int j = 0; j < 4; ++j)
          if (q0 + j < nparts && q0 + j != part) mt = fmaxf(mt, mq[j]);
      }
      f32x16 own[NDB];
#pragma unroll
      for (int db = 0; db < NDB; ++db) {
        own[db] = oacc[qb][db];
        oacc[qb][db] = (f32x16){};
      }
      float l = 0.f;
      for (int q0 = 0; q0 < nparts; q0 += CH) {
        f32x4 ml[CH], x[CH][4 * NDB];
#pragma unroll
        for (int j = 0; j < CH; ++j) {
          const int qq = min(q0 + j, nparts - 1);
          ml[j] = ld_ws(voff(qq, qb * NVB + 4 * NDB));
#pragma unroll
          for (int v = 0; v < 4 * NDB; ++v) x[j][v] = ld_ws(voff(qq, qb * NVB + v));
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
            for (int i = 0; i < 16; ++i)
              oacc[qb][db][i] = __builtin_fmaf(mine ? own[db][i] : x[j][4 * db + i / 4][i % 4], a, oacc[qb][db][i]);
        }
      }
      lrow[qb] = l;
    }
  }

  // ---- normalise, store
#pragma unroll
  for (int qb = 0; qb < QB; ++qb) {
    const float inv = lrow[qb] > 0.f ? 1.f / lrow[qb] : 0.f;
    const int qrow = qw0 + 32 * qb + l32;
    // log-sum-exp in natural log: (offset + log2 of the sum) * ln 2; a row
    // that saw no key gets -inf (its output is zero)
    if constexpr ((OPT & 32) != 0) {
      if (qrow < Sq && hh == 0)
        p.lse[(int64_t)bh * Sq + qrow] =
            lrow[qb] > 0.f ? (mb[qb] + __builtin_amdgcn_logf(lrow[qb])) * 0.6931471805599453f : -INFINITY;
    }
    if (qrow < Sq) {
      uint16_t* orow = og + row_off(qrow, p.o_g, p.o_s);
#pragma unroll
      for (int db = 0; db < NDB; ++db) {
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const int d = 32 * db + 8 * g + 4 * hh;
          if (d < D) {
            u32x2 w;
            w[0] = Elt<T>::pack(oacc[qb][db][4 * g + 0] * inv, oacc[qb][db][4 * g + 1] * inv);
            w[1] = Elt<T>::pack(oacc[qb][db][4 * g + 2] * inv, oacc[qb][db][4 * g + 3] * inv);
            if (ELEM)
              st_cols16x4(orow + d, w, D - d, p.elem_rows);
            else
              *(u32x2*)(orow + d) = w;
          }
        }
      }
    }
  }
}

// Launch one instance: grid = B*H*ceil(Sq/BQ) workgroups of NW waves.
// Key split plan: only when the query blocks leave CUs idle (fewer blocks
// than CUs), into enough parts for up to two workgroups per CU
// (as many as fit: one at head dims above 128), each part at least
// kMinTiles16 key tiles long, and at most 32 parts.  When every wave of a
// block holds rows, the last part's waves each merge their own rows: then
// at most 8 parts from a 192-wide output up (a wave reads every other part's
// O back, one part per memory round trip at those widths; measured on
// MI355X, bf16 grouped-query decode over 8 K/V heads (8 packed blocks):
// D = 256, 16384 keys, 2 / 8 / 32 / 64 parts 428 / 178 / 306 / 592 us with
// that merge).  Blocks with rows in fewer waves (`spread`: decode, packed
// query groups) merge across the whole workgroup and keep the cap of 32.
// Causal launches: below.  Returns the part count (1: no split).
constexpr int kMinTiles16 = 4;
inline int split_parts16(int n, int ntiles, int wg_per_cu, int cus, bool causal, int dp, bool spread,
                         int ntiles_min) {
  if (n <= 0 || n >= cus) return 1;
  int parts = (wg_per_cu < 2 ? wg_per_cu : 2) * cus / n;
  if (causal) {
    // ntiles: the last block's sweep (to its last row), ntiles_min the
    // first's; every part keeps a tile, the longest at least 16 (a causal row
    // sees a key in a part's first tile or none of the part's keys, and then
    // has no weight in the merge); only where most CUs idle or sweeps are long
    if (n * 2 > cus && ntiles < 64) return 1;
    if (parts > ntiles / 16) parts = ntiles / 16;
    if (parts > ntiles_min) parts = ntiles_min;
    if (parts > 8) parts = 8;
    return parts >= 2 ? parts : 1;
  }
  if (parts > ntiles / kMinTiles16) parts = ntiles / kMinTiles16;
  const int cap = dp >= 192 && !spread ? 8 : 32;
  if (parts > cap) parts = cap;
  return parts >= 2 ? parts : 1;
}

// Launch one instance: grid = B*H*ceil(Sq/BQ) workgroups of NW waves, times
// the part count of split blocks.
template <typename T, int DK, int NW, int QB, int BK, int OCC, bool CAUSAL, bool PRESCALE,
          int OPT = 0>
hipError_t launch_mfma16_cfg(const FwdParams& p0, hipStream_t stream) {
  constexpr int DP = (DK + 31) / 32 * 32;
  constexpr int BQ = NW * QB * 32;
  FwdParams p = p0;
  p.n_qblk = (p.Sq + BQ - 1) / BQ;
  p.n_wg = p.B * p.H * p.n_qblk;
  if (p.n_wg == 0) return hipSuccess;
  const int n = p.n_wg;
  // waves per block that hold query rows (a single block shorter than BQ has fewer)
  const int nwl = p.n_qblk > 1 ? NW : (p.Sq + QB * 32 - 1) / (QB * 32) < NW ? (p.Sq + QB * 32 - 1) / (QB * 32) : NW;
  SplitArgs sa = {n, 1, nullptr, nullptr, nwl};
  // the training forward (OPT bit 5) runs every block whole
  const int kmax = CAUSAL && (int64_t)p.n_qblk * BQ < p.Sk ? p.n_qblk * BQ : p.Sk;  // the last block's keys
  const int kmin = CAUSAL && BQ < p.Sk ? BQ : p.Sk;                                 // the first block's
  const int parts = (OPT & 32) ? 1
                               : split_parts16(n, (kmax + BK - 1) / BK, OCC, device_cus(), CAUSAL, DP, nwl < NW,
                                               (kmin + BK - 1) / BK);
  if (parts >= 2) {
    // every block is split; one key range of all of them takes part_bytes
    const size_t part_bytes = (size_t)n * nwl * QB * split_vectors(DP) * 64 * sizeof(f32x4);
    f32x4* ws = nullptr;
    int* cnt = nullptr;
    const int fit = bind_exchange(p, parts, part_bytes, 2 * n * nwl, &ws, &cnt);
    if (fit >= 2) sa = SplitArgs{0, fit, ws, cnt, nwl};
  }
  if (p.dry) return hipSuccess;
  const int nwg = sa.nfull + (n - sa.nfull) * sa.nparts;
  hipLaunchKernelGGL((attn_fwd_mfma16<T, DK, DP, NW, QB, BK, OCC, CAUSAL, PRESCALE, OPT>), dim3(nwg),
                     dim3(NW * 64), 0, stream, p, sa);
  return hipGetLastError();
}

}  // namespace cmpext3
