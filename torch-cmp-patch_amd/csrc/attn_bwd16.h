// Backward pass of the fused attention, fp16 / bf16 on gfx950
// (v_mfma_f32_32x32x16_{f16,bf16}), head-dim buckets 64, 128, 192 and 256.
//
// Given Q, K, V, the forward output O, its gradient dO and the forward's row
// log-sum-exp (natural log, written by the forward's training variant), with
// P = softmax(S), S = scale * Q K^T (causal: top-left, key j visible to
// query i iff j <= i):
//   Delta_i = sum_d dO_id O_id                     (attn_bwd_delta)
//   dV = P^T dO,  dK = scale * dS^T Q              (attn_bwd_dkdv, per key block)
//   dQ = scale * dS K                              (attn_bwd_dq, per query block)
//   with dP = dO V^T and dS = P * (dP - Delta).
// P is recomputed from the scores and the saved log-sum-exp, so nothing of
// size Sq x Sk is stored.  The two gradient kernels each own their output rows
// outright (no atomics), so the results are bit-identical from run to run;
// where a sweep is split over several workgroups (few blocks for the CUs),
// their fp32 partials go to a caller workspace and attn_bwd_part_sum adds
// them in a fixed order.  The reference is forward-only (its patch hands
// calls with live autograd to stock torch, cmpext3/__init__.py:115-125);
// this is the gradient of the same forward, checked against the float64
// restatement in oracle/sdpa_oracle.py (sdpa_bwd_np).
//
// Layout: one 32 x 32 MFMA accumulator holds scores for 32 queries x 32 keys.
// The dK/dV kernel keeps lane = key: S = Q K^T and dP = dO V^T take their B
// operand (8 head-dim values of the lane's key) from registers loaded once,
// their A operand (query rows) from the LDS tile; P and dS then sit in the
// lanes exactly as the B operand of dV^T = dO^T P and dK^T = Q^T dS needs them
// (8 consecutive queries per lane, thanks to the bit-permuted row feed), and
// dO^T / Q^T come from the same LDS tiles through ds_read_b64_tr_b16.  The dQ
// kernel mirrors the forward: lane = query, S^T = K Q^T, dP^T = V dO^T,
// dQ^T = K^T dS^T.  A negative scale is folded into the sign of the operand
// held in registers (K in dK/dV, Q in dQ), and the signed scale multiplies the
// result.  Grouped-query K/V (Hkv heads shared by H / Hkv query heads each):
// a dK/dV workgroup sweeps the query tiles of every query head of its group
// (or its part of that sequence), so the group's contributions are summed in
// registers.
#pragma once

#include "attn_fwd_pipe16.h"

namespace cmpext3 {

struct BwdParams {
  const void* q;
  const void* k;
  const void* v;
  const void* o;
  const void* dout;
  const float* lse;  // [B*H, Sq] row log-sum-exp of scale * Q K^T (natural log)
  void* dq;
  void* dk;
  void* dv;
  float* delta;      // [B*H, Sq] workspace: sum_d dO * O per row
  // element strides of dims {batch, head, seq}; head-dim stride is 1
  int64_t q_b, q_h, q_s, k_b, k_h, k_s, v_b, v_h, v_s, o_b, o_h, o_s, do_b, do_h, do_s;
  int64_t dq_b, dq_h, dq_s, dk_b, dk_h, dk_s, dv_b, dv_h, dv_s;
  int B, H, Sq, Sk, D;
  int Hkv;          // K/V heads (dk, dv have Hkv heads); query head h uses K/V head h / group
  int group;        // H / Hkv
  int n_blk;        // key blocks (dK/dV, per K/V head) or query blocks (dQ, per query head)
  int n_wg;         // workgroups launched = B * H * n_blk (dK/dV: times nsplit)
  float c;          // |scale| * log2(e)
  float scale;      // signed scale: dK = scale * dS^T Q, dQ = scale * dS K
  uint32_t sign;    // 0x80008000 when scale < 0 (XORed into K or Q words), else 0
  // optional attention mask, as in FwdParams (element strides over {batch,
  // head, query}, unit key stride, kind MASK_*; MASK_NONE = none)
  const void* mask;
  int64_t m_b, m_h, m_q;
  int mask_kind;
  // split sweeps: nsplit > 1 dK/dV workgroups per key block, each leaving
  // fp32 partial dK / dV rows in `part` ([nsplit][B * Hkv][Sk][D] for dK, then
  // the same for dV); nsplit_q > 1 dQ workgroups per query block, partial dQ
  // rows in `part_q` ([nsplit_q][B * H][Sq][D]); attn_bwd_part_sum adds them
  int nsplit, nsplit_q;
  float* part;
  float* part_q;
  // f16/bf16, non-causal: with nfull > 0 only the blocks past the first nfull
  // (the last, partial round of workgroup slots) are split, and their
  // partials are block-indexed: [nsplit][blocks - nfull][128][D] (likewise
  // nfull_q for dQ)
  int nfull, nfull_q;
};

// Parts per block of a gradient sweep (1 = unsplit).  With too few blocks
// (n_wg) for the CU slots the kernel's occupancy allows (one 4-wave workgroup
// per wave per SIMD), each block's sweep is cut into contiguous parts whose
// fp32 partials are summed afterwards: non-causal, as many parts as fill one
// round of slots; causal, enough for two rounds, so that longest-first
// dispatch pairs long parts with short ones (causal sweeps' lengths run from
// one tile to all of them).  At most 8 parts, each at least 4 tiles of the
// longest sweep (`tiles`).
inline int split_sweep(int64_t n_wg, int occ, int cus, bool causal, int64_t tiles) {
  const int64_t slots = (int64_t)cus * occ;
  const int64_t want = causal ? 2 * slots : slots;
  if (n_wg <= 0 || n_wg * 2 > want) return 1;
  int64_t ns = causal ? (want + n_wg - 1) / n_wg : want / n_wg;
  if (ns > 8) ns = 8;
  if (ns > tiles / 4) ns = tiles / 4;
  return ns >= 2 ? (int)ns : 1;
}

// Split plan of a backward launch and its workspace: the dK/dV partials
// (2 x ns_kv x B x Hkv x Sk x D floats), then the dQ partials (ns_q x B x H
// x Sq x D floats).
struct BwdSplit {
  int ns_kv = 1, ns_q = 1;
  int nfull_kv = 0, nfull_q = 0;  // split tails: whole blocks before them
  size_t kv_bytes(int B, int Hkv, int Sk, int D) const {
    if (ns_kv < 2) return 0;
    if (nfull_kv > 0)
      return (size_t)2 * ns_kv * ((int64_t)B * Hkv * ((Sk + 127) / 128) - nfull_kv) * 128 * D * sizeof(float);
    return (size_t)2 * ns_kv * B * Hkv * Sk * D * sizeof(float);
  }
  size_t q_bytes(int B, int H, int Sq, int D) const {
    if (ns_q < 2) return 0;
    if (nfull_q > 0) return (size_t)ns_q * ((int64_t)B * H * ((Sq + 127) / 128) - nfull_q) * 128 * D * sizeof(float);
    return (size_t)ns_q * B * H * Sq * D * sizeof(float);
  }
};

// Split tail of a non-causal grid of n equal sweeps that fills more than one
// but not a whole number of rounds of one workgroup per CU, within the occ
// workgroups per CU the kernel allows (SDXL self-attention: 640 blocks at
// three per CU): the blocks past the whole rounds are cut into parts, one
// per CU, so every CU holds the same work (as the forward's key split does).
// Returns the parts (1 = none) and sets *nfull.
inline int split_tail(int64_t n, int occ, int cus, int64_t tiles, int* nfull) {
  *nfull = 0;
  if (cus <= 0) return 1;
  const int64_t full = n / cus, rem = n - full * cus;
  if (full == 0 || rem == 0 || full + 1 > occ) return 1;
  int64_t ns = cus / rem;
  if (ns > 8) ns = 8;
  if (ns > tiles / 8) ns = tiles / 8;
  if (ns < 2) return 1;
  *nfull = (int)(full * cus);
  return (int)ns;
}

// fp32 partial rows of a split sweep ([ns][rows][D], rows = B x heads x S)
// and where their sum goes: T rows with element strides {batch, head, seq},
// times `mul`.
struct PartSum {
  const float* part;
  void* out;
  int64_t ob, oh, os;
  int64_t rows;
  int heads, S, D, ns;
  float mul;
};

// LDS row stride (halves) of the Q/dO and K/V tiles: rows padded by 16 bytes,
// by 48 at D = 128 (fewer bank conflicts there: dK/dV 285 -> 277 us and dQ
// 125 -> 123 us on causal bf16 [4,16,2048,128]; no change at D = 64).
// Waves per SIMD of the two gradient kernels: D > 128 holds the dK and dV
// accumulators alone in 2 * DK registers per lane, so those run one wave.
constexpr int bwd_lds_stride(int dk) { return dk + (dk == 128 ? 24 : 8); }

// Mask element size in bytes.
__device__ __forceinline__ int mask_bytes(int kind) { return kind == MASK_BOOL ? 1 : kind == MASK_F32 ? 4 : 2; }

// One mask element as an exp2-domain addend: -inf for a dropped pair (bool
// zero), value * log2(e) for additive masks.  `off` is a byte offset into the
// descriptor's range (reads past it return zero).
__device__ __forceinline__ float mask_elem(__amdgpu_buffer_rsrc_t rs, int off, int kind) {
  if (kind == MASK_BOOL) return __builtin_amdgcn_raw_buffer_load_b8(rs, off, 0, 0) ? 0.f : -INFINITY;
  if (kind == MASK_F32) return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rs, off, 0, 0)) * kLog2e;
  const uint32_t w = __builtin_amdgcn_raw_buffer_load_b16(rs, off, 0, 0);
  const float f = kind == MASK_F16 ? (float)__builtin_bit_cast(_Float16, (uint16_t)w)
                                   : __uint_as_float(w << 16);
  return f * kLog2e;
}

// ---- Delta_i = sum_d dO_id * O_id (fp32), 8 lanes per row
template <typename T>
__global__ void __launch_bounds__(256) attn_bwd_delta(const BwdParams p) {
  const int sub = thread_x() & 7;
  const int64_t g = (int64_t)block_x() * 32 + (thread_x() >> 3);  // row over B*H*Sq
  const bool live = g < (int64_t)p.B * p.H * p.Sq;
  float acc = 0.f;
  if (live) {
    const int64_t bh = g / p.Sq;
    const int i = (int)(g - bh * p.Sq);
    const int b = (int)(bh / p.H), h = (int)(bh - (int64_t)b * p.H);
    const uint16_t* orow = (const uint16_t*)p.o + b * p.o_b + h * p.o_h + (int64_t)i * p.o_s;
    const uint16_t* drow = (const uint16_t*)p.dout + b * p.do_b + h * p.do_h + (int64_t)i * p.do_s;
    for (int c8 = sub; 8 * c8 < p.D; c8 += 8) {
      const u32x4 a = *(const u32x4*)(orow + 8 * c8);
      const u32x4 d = *(const u32x4*)(drow + 8 * c8);
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        const f32x2 x = Elt<T>::unpack(a[w]), y = Elt<T>::unpack(d[w]);
        acc = __builtin_fmaf(x[0], y[0], acc);
        acc = __builtin_fmaf(x[1], y[1], acc);
      }
    }
  }
  acc += __shfl_xor(acc, 1, 8);
  acc += __shfl_xor(acc, 2, 8);
  acc += __shfl_xor(acc, 4, 8);
  if (live && sub == 0) p.delta[g] = acc;
}

// One 32-row tile (rows r0.., DK columns) of a [rows, D] matrix into registers,
// 16-byte chunks spread over the 256 threads; rows past `nrows` read as zero
// (buffer bounds), chunks past D are zeroed.
template <int DK>
struct TileLoader {
  static constexpr int KCH = DK / 8;
  static constexpr int N = 32 * KCH / 256;  // chunks per thread
  static_assert(32 * KCH % 256 == 0, "whole chunks per thread");
  int voff[N], loff[N];
  bool zero[N];
  __device__ __forceinline__ void init(int tid, int64_t row_stride, int D, int RS) {
#pragma unroll
    for (int it = 0; it < N; ++it) {
      const int ci = it * 256 + tid, r = ci / KCH, c8 = ci - r * KCH;
      voff[it] = (int)(r * row_stride * 2) + 16 * c8;
      loff[it] = r * RS + 8 * c8;
      zero[it] = 8 * c8 >= D;
    }
  }
  __device__ __forceinline__ void load(__amdgpu_buffer_rsrc_t rs, int soff, u32x4 (&x)[N]) const {
#pragma unroll
    for (int it = 0; it < N; ++it)
      x[it] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rs, voff[it], soff, 0));
  }
  __device__ __forceinline__ void store(uint16_t* dst, const u32x4 (&x)[N]) const {
#pragma unroll
    for (int it = 0; it < N; ++it) *(u32x4*)(dst + loff[it]) = zero[it] ? (u32x4){0u, 0u, 0u, 0u} : x[it];
  }
};

// A-operand fragment of X^T for a 16-row slice of a row-major LDS tile
// (row = query or key, column = head dim): 8 consecutive rows of one column.
__device__ __forceinline__ u32x4 tr_frag(const uint16_t* base, int off0, int off1) {
  const uint2 lo = lds_tr16_b64(base + off0);
  const uint2 hi = lds_tr16_b64(base + off1);
  return (u32x4){lo.x, lo.y, hi.x, hi.y};
}

// Store a [32 rows x DP] accumulator set (C layout: lane = row l32, register
// 4g + j of block db = column 32 db + 8 g + 4 hh + j) times `mul` as T.
template <typename T, int NDB>
__device__ __forceinline__ void store_rows(uint16_t* base, int64_t row_stride, int row, int nrows, int D, int hh,
                                           const f32x16 (&acc)[NDB], float mul) {
  if (row >= nrows) return;
  uint16_t* dst = base + (int64_t)row * row_stride;
#pragma unroll
  for (int db = 0; db < NDB; ++db)
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const int d = 32 * db + 8 * g + 4 * hh;
      if (d < D) {
        u32x2 w;
        w[0] = Elt<T>::pack(acc[db][4 * g + 0] * mul, acc[db][4 * g + 1] * mul);
        w[1] = Elt<T>::pack(acc[db][4 * g + 2] * mul, acc[db][4 * g + 3] * mul);
        *(u32x2*)(dst + d) = w;
      }
    }
}

// The same accumulator set unscaled, as fp32 rows of D floats (row = lane's
// key; rows past nrows are not stored).
template <int NDB>
__device__ __forceinline__ void store_rows_f32(float* base, int row, int nrows, int D, int hh,
                                               const f32x16 (&acc)[NDB]) {
  if (row >= nrows) return;
  float* dst = base + (int64_t)row * D;
#pragma unroll
  for (int db = 0; db < NDB; ++db)
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const int d = 32 * db + 8 * g + 4 * hh;
      if (d < D)
        *(f32x4*)(dst + d) =
            (f32x4){acc[db][4 * g + 0], acc[db][4 * g + 1], acc[db][4 * g + 2], acc[db][4 * g + 3]};
    }
}

// ---- dK, dV for one block of 128 keys (4 waves x 32 keys), sweeping the
// query tiles (32 rows of Q, dO, lse, Delta) through double-buffered LDS.
// Waves per SIMD: D <= 64: 3 (masked with V parked in LDS; 4 spilled
// registers), 2 causal; D <= 128: 2 with V parked in LDS (the causal and the
// masked variants spill 8 registers and are still 12-20% faster than at 1),
// 1 masked causal (its K/V operands and dK/dV accumulators alone take 192
// registers); D > 128: 1, with V parked in LDS.
template <typename T, int DK, bool CAUSAL, bool MASK>
__global__ void __launch_bounds__(256)
__attribute__((amdgpu_waves_per_eu(DK <= 64 ? (CAUSAL ? 2 : 3) : (DK > 128 || (MASK && CAUSAL)) ? 1 : 2)))
attn_bwd_dkdv(const BwdParams p) {
  constexpr int BQ = 32, BKV = 128;
  constexpr int RS = bwd_lds_stride(DK);  // LDS row stride (halves)
  constexpr int NKS = DK / 16, NDB = DK / 32;
  static_assert(DK % 32 == 0, "head-dim bucket");
  __shared__ __attribute__((aligned(16))) uint16_t lds[2 * 2 * BQ * RS];  // [slot][Q, dO][row][col]
  // The V operands live in LDS instead of registers where that buys a wave
  // per SIMD: D > 64 (32 fewer VGPRs, two waves instead of one; dK/dV
  // 349 -> 268 us on bf16 [4,16,2048,128], 275 -> 241 us causal, masked
  // backward 603 -> 481 us) and D <= 64 masked non-causal (three waves
  // instead of two: masked SDXL-shape backward 913 -> 616 us).  Each lane
  // reads back only what it wrote, so no barrier orders the parking stores.
  // Not for masked causal 64 < D <= 128 (32 spilled registers at two waves)
  // or causal D <= 64 (three waves with V parked measured slower: 301 -> 327
  // us).  Above D = 128 always: the K operands (DK / 4 registers) and the
  // two accumulators (2 * DK) leave little of one wave's 512 registers.
  constexpr bool VLDS = DK > 128 ? true : DK > 64 ? !(MASK && CAUSAL) : (MASK && !CAUSAL);
  constexpr int RSV = DK + 8;
  __shared__ __attribute__((aligned(16))) uint16_t vpark[VLDS ? BKV * RSV : 8];
  // [slot][-lse2 / c, -Delta][row]: the starting values of the S and dP
  // accumulators, so that the MFMAs leave S - lse2 / c and dP - Delta
  __shared__ __attribute__((aligned(16))) float lsd[2][2][BQ];

  const int tid = thread_x(), wave = tid >> 6, lane = tid & 63, l32 = lane & 31, hh = lane >> 5;
  // (batch, K/V head) and key block; split sweeps: (block, part) pairs as
  // virtual blocks.  Causal: longest sweeps first (kv_tile).  (The divisions
  // run on the vector unit: readfirstlane keeps the indices, and the per-head
  // address arithmetic of the sweep, in scalar registers.)
  int ns = p.nsplit > 1 ? p.nsplit : 1;
  int bhk, kb, part, sb = -1;  // sb: index among a split tail's blocks
  if (!CAUSAL && p.nfull > 0) {
    // split tail: the first nfull workgroups take whole blocks, the rest
    // ns-way parts of the remaining blocks
    const int w = block_x();
    int tile = w;
    part = 0;
    if (w >= p.nfull) {
      const int r = w - p.nfull;
      tile = p.nfull + r / ns;
      part = r - (tile - p.nfull) * ns;
      sb = tile - p.nfull;
    } else {
      ns = 1;
    }
    int bh0, kb0;
    kv_tile(tile, p.B * p.Hkv, p.n_blk, false, bh0, kb0);
    bhk = __builtin_amdgcn_readfirstlane(bh0);
    kb = __builtin_amdgcn_readfirstlane(kb0);
  } else {
    int bh0, vb;
    kv_tile(block_x(), p.B * p.Hkv, p.n_blk * ns, CAUSAL, bh0, vb);
    bhk = __builtin_amdgcn_readfirstlane(bh0);
    vb = __builtin_amdgcn_readfirstlane(vb);
    kb = __builtin_amdgcn_readfirstlane(vb / ns);
    part = vb - kb * ns;
  }
  const int b = __builtin_amdgcn_readfirstlane(bhk / p.Hkv), hk = bhk - b * p.Hkv;
  const int Sq = p.Sq, Sk = p.Sk, D = p.D;
  const int kw0 = kb * BKV + wave * 32;  // first key of this wave
  const int key = kw0 + l32;             // this lane's key

  // B operands held for the whole sweep: 8 head-dim values of this lane's key
  const uint16_t* kg = (const uint16_t*)p.k + b * p.k_b + hk * p.k_h;
  const uint16_t* vg = (const uint16_t*)p.v + b * p.v_b + hk * p.v_h;
  u32x4 kf[NKS], vf[VLDS ? 1 : NKS];
  uint16_t* const vrow = vpark + (wave * 32 + l32) * RSV + 8 * hh;  // this lane's parked V
#pragma unroll
  for (int s = 0; s < NKS; ++s) {
    const int d = 16 * s + 8 * hh;
    u32x4 x = {0u, 0u, 0u, 0u}, y = {0u, 0u, 0u, 0u};
    if (key < Sk && d < D) {
      x = *(const u32x4*)(kg + (int64_t)key * p.k_s + d);
      y = *(const u32x4*)(vg + (int64_t)key * p.v_s + d);
    }
    kf[s] = x ^ p.sign;
    if constexpr (VLDS)
      *(u32x4*)(vrow + 16 * s) = y;
    else
      vf[s] = y;
  }

  TileLoader<DK> lq, ldo;
  lq.init(tid, p.q_s, D, RS);
  ldo.init(tid, p.do_s, D, RS);

  // fragment read offsets: A = query rows (bit-permuted), A = X^T slices
  int a_rd[NKS];
  {
    const int r = perm_row(l32);
#pragma unroll
    for (int s = 0; s < NKS; ++s) a_rd[s] = r * RS + 16 * s + 8 * hh;
  }
  const int jj = lane & 15, gg = lane >> 4;
  int t_rd[NDB][2];
#pragma unroll
  for (int db = 0; db < NDB; ++db)
#pragma unroll
    for (int half = 0; half < 2; ++half)
      t_rd[db][half] = (8 * (gg >> 1) + (jj >> 2) + 4 * half) * RS + 32 * db + 16 * (gg & 1) + 4 * (jj & 3);

  f32x16 dva[NDB], dka[NDB];
#pragma unroll
  for (int db = 0; db < NDB; ++db) dva[db] = dka[db] = (f32x16){};

  // The sweep: query tiles t0 .. t1-1 of each query head of the group, as one
  // sequence of nj tiles, of which this workgroup takes [jb, je) (all of it
  // unless the sweep is split).  (fg, ft) is the head and tile of the next
  // fetch, (cg, ct) those of the tile being computed: running counters.
  const int t0 = CAUSAL ? kb * (BKV / BQ) : 0;  // query tiles before the block see none of its keys
  const int t1 = (Sq + BQ - 1) / BQ;
  const int nt = t1 > t0 ? t1 - t0 : 0;
  const int nj = nt * p.group;
  const int jb = (int)((int64_t)part * nj / ns), je = (int)((int64_t)(part + 1) * nj / ns);
  const int jg0 = nt > 0 ? jb / nt : 0;
  u32x4 xq[TileLoader<DK>::N], xd[TileLoader<DK>::N];
  float xl = -INFINITY, xdl = 0.f;  // raw lse / Delta of the fetched rows
  const float inv_c = 1.f / p.c;    // c > 0 (the caller floors it for tiny |scale|)
  const int h0 = hk * p.group;      // first query head of the group
  int fg = jg0, ft = t0 + (jb - jg0 * nt);
  auto fetch = [&]() {
    const int h = h0 + fg;
    const uint16_t* qg = (const uint16_t*)p.q + b * p.q_b + h * p.q_h;
    const uint16_t* dog = (const uint16_t*)p.dout + b * p.do_b + h * p.do_h;
    const __amdgpu_buffer_rsrc_t qrs = uniform_rsrc(qg, ((int64_t)(Sq - 1) * p.q_s + D) * 2);
    const __amdgpu_buffer_rsrc_t dors = uniform_rsrc(dog, ((int64_t)(Sq - 1) * p.do_s + D) * 2);
    const int q0 = ft * BQ;
    lq.load(qrs, (int)(q0 * p.q_s * 2), xq);
    ldo.load(dors, (int)(q0 * p.do_s * 2), xd);
    // this head's lse / Delta rows; used only in put(), so the loads are not
    // waited for before the current tile's products
    const int64_t hoff = ((int64_t)b * p.H + h) * Sq;
    if (tid < BQ) {
      const int row = q0 + tid;
      // rows past Sq: P = 0
      xl = -INFINITY;
      xdl = 0.f;
      if (row < Sq) {
        xl = p.lse[hoff + row];
        xdl = p.delta[hoff + row];
      }
    }
    if (++ft == t1) {
      ft = t0;
      ++fg;
    }
  };
  auto put = [&](int slot) {
    uint16_t* base = lds + slot * 2 * BQ * RS;
    lq.store(base, xq);
    ldo.store(base + BQ * RS, xd);
    if (tid < BQ) {
      // rows that saw no key in the forward (lse = -inf): P = 0
      lsd[slot][0][tid] = xl > -INFINITY ? -(xl * kLog2e) * inv_c : -INFINITY;
      lsd[slot][1][tid] = -xdl;
    }
  };

  const float c = p.c;
  // lane = key, registers = head-dim columns
  uint16_t* dkg = (uint16_t*)p.dk + b * p.dk_b + hk * p.dk_h;
  uint16_t* dvg = (uint16_t*)p.dv + b * p.dv_b + hk * p.dv_h;
  // the result: gradients, or this part's fp32 partials (dK unscaled)
  auto finish = [&]() {
    if (ns > 1 && sb >= 0) {  // split tail: block-indexed rows
      const int64_t nsb = (int64_t)p.B * p.Hkv * p.n_blk - p.nfull;
      float* const pk = p.part + ((int64_t)part * nsb + sb) * 128 * D;
      const int kl = key - kb * 128;
      store_rows_f32<NDB>(pk, kl, Sk - kb * 128, D, hh, dka);
      store_rows_f32<NDB>(pk + ns * nsb * 128 * D, kl, Sk - kb * 128, D, hh, dva);
    } else if (ns > 1) {
      const int64_t rows = (int64_t)p.B * p.Hkv * Sk;
      float* const pk = p.part + ((int64_t)part * p.B * p.Hkv + bhk) * Sk * D;
      store_rows_f32<NDB>(pk, key, Sk, D, hh, dka);
      store_rows_f32<NDB>(pk + ns * rows * D, key, Sk, D, hh, dva);
    } else {
      store_rows<T, NDB>(dvg, p.dv_s, key, Sk, D, hh, dva, 1.f);
      store_rows<T, NDB>(dkg, p.dk_s, key, Sk, D, hh, dka, p.scale);
    }
  };
  if (je == jb) {  // no query of this range sees the block (causal): zeros
    finish();
    return;
  }
  // (the loop is entered only past put(0), whose waits cover the operand
  // loads above: no load of those is outstanding inside the loop)
  fetch();
  put(0);
  lds_barrier();
  int cg = jg0, ct = t0 + (jb - jg0 * nt);
  for (int j = jb; j < je; ++j) {
    const int slot = (j - jb) & 1;
    if (j + 1 < je) fetch();
    const int q0 = ct * BQ;
    // causal: a tile whose last query precedes this wave's first key adds nothing
    if (!CAUSAL || q0 + BQ - 1 >= kw0) {
      const uint16_t* qs = lds + slot * 2 * BQ * RS;
      const uint16_t* dos = qs + BQ * RS;
      // attention mask of this tile as exp2-domain addends, one element per
      // (query row of register r, this lane's key); lanes of one half read
      // consecutive keys of one row
      float madd[16];
      if (MASK) {
        const int kind = p.mask_kind, mes = mask_bytes(kind);
        const int h = h0 + cg;
        const __amdgpu_buffer_rsrc_t mrs = uniform_rsrc(
            (const char*)p.mask + (b * p.m_b + h * p.m_h) * mes, ((int64_t)(Sq - 1) * p.m_q + (Sk + 7) / 8 * 8) * mes);
        if (p.m_q == 0 || Sq == 1) {
          // the same row for every query (key padding, per-head biases): one
          // element per lane serves all 16 rows
          const float a = mask_elem(mrs, key * mes, kind);
#pragma unroll
          for (int r = 0; r < 16; ++r) madd[r] = a;
        } else {
#pragma unroll
          for (int r = 0; r < 16; ++r)
            madd[r] = mask_elem(mrs, (int)(((int64_t)(q0 + acc_key(r, hh)) * p.m_q + key) * mes), kind);
        }
      }
      // register r holds query q0 + acc_key(r, hh): two runs of 8 consecutive rows
      f32x16 s, dp;
#pragma unroll
      for (int run = 0; run < 2; ++run)
#pragma unroll
        for (int h4 = 0; h4 < 2; ++h4) {
          const f32x4 a = *(const f32x4*)&lsd[slot][0][16 * run + 8 * hh + 4 * h4];
          const f32x4 d = *(const f32x4*)&lsd[slot][1][16 * run + 8 * hh + 4 * h4];
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            s[8 * run + 4 * h4 + i] = a[i];
            dp[8 * run + 4 * h4 + i] = d[i];
          }
        }
#pragma unroll
      for (int st = 0; st < NKS; ++st) s = Elt<T>::mma(*(const u32x4*)(qs + a_rd[st]), kf[st], s);
#pragma unroll
      for (int st = 0; st < NKS; ++st) {
        u32x4 vb;
        if constexpr (VLDS)
          vb = *(const u32x4*)(vrow + 16 * st);
        else
          vb = vf[st];
        dp = Elt<T>::mma(*(const u32x4*)(dos + a_rd[st]), vb, dp);
      }
      // s = S - lse2 / c, dp = dP - Delta
      float x[16];
#pragma unroll
      for (int r = 0; r < 16; ++r) x[r] = MASK ? __builtin_fmaf(s[r], c, madd[r]) : s[r] * c;
      // causal diagonal tile: one wave-uniform branch around all 16 checks
      if (CAUSAL && q0 < kw0 + 31) {
#pragma unroll
        for (int r = 0; r < 16; ++r)
          if (key > q0 + acc_key(r, hh)) x[r] = -INFINITY;
      }
      u32x4 pp[2], ps[2];
#pragma unroll
      for (int ks = 0; ks < 2; ++ks)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          float pv[2];
#pragma unroll
          for (int u = 0; u < 2; ++u) pv[u] = fast_exp2(x[8 * ks + 2 * e + u]);
          pp[ks][e] = Elt<T>::pack(pv[0], pv[1]);
          ps[ks][e] = Elt<T>::pack(pv[0] * dp[8 * ks + 2 * e], pv[1] * dp[8 * ks + 2 * e + 1]);
        }
      // dV^T += dO^T P, dK^T += Q^T dS (16 queries per k-step)
#pragma unroll
      for (int ks = 0; ks < 2; ++ks)
#pragma unroll
        for (int db = 0; db < NDB; ++db) {
          const uint16_t* dsl = dos + 16 * ks * RS;
          dva[db] = Elt<T>::mma(tr_frag(dsl, t_rd[db][0], t_rd[db][1]), pp[ks], dva[db]);
          const uint16_t* qsl = qs + 16 * ks * RS;
          dka[db] = Elt<T>::mma(tr_frag(qsl, t_rd[db][0], t_rd[db][1]), ps[ks], dka[db]);
        }
    }
    if (j + 1 < je) put(slot ^ 1);
    lds_barrier();
    if (++ct == t1) {
      ct = t0;
      ++cg;
    }
  }
  finish();
}

// ---- Sums of split sweeps' partials, in part order (the same result on every
// run): vector i4 (4 columns) of one or two outputs (b.out null: one).
template <typename T>
__device__ __forceinline__ void part_sum_store(const PartSum& a, int64_t i4) {
  const int64_t row = i4 * 4 / a.D;
  const int d = (int)(i4 * 4 - row * a.D);
  const int64_t bh = row / a.S;
  const int s = (int)(row - bh * a.S);
  const int b = (int)(bh / a.heads), h = (int)(bh - (int64_t)b * a.heads);
  const f32x4* const pk = (const f32x4*)a.part + i4;
  const int64_t step = a.rows * a.D / 4;  // one part's vectors
  f32x4 x = pk[0];
  for (int q = 1; q < a.ns; ++q) x += pk[q * step];
  x = x * a.mul;
  T* const dst = (T*)a.out + b * a.ob + h * a.oh + (int64_t)s * a.os + d;
  if constexpr (sizeof(T) == 4) {
    *(f32x4*)dst = x;
  } else {
    u32x2 w;
    w[0] = Elt<T>::pack(x[0], x[1]);
    w[1] = Elt<T>::pack(x[2], x[3]);
    *(u32x2*)dst = w;
  }
}

template <typename T>
__global__ void __launch_bounds__(256) attn_bwd_part_sum(const PartSum a, const PartSum b) {
  const int64_t i4 = (int64_t)block_x() * 256 + thread_x();
  if (i4 >= a.rows * a.D / 4) return;
  part_sum_store<T>(a, i4);
  if (b.out) part_sum_store<T>(b, i4);
}

// ---- Sums of a split tail's block-indexed partials ([ns][blocks][128][D]),
// in part order: split block sb is logical block nfull + sb, mapped to its
// (head, block) as the gradient kernel maps it; rows past Sk (Sq) are not
// stored.  KV: dK (times the signed scale) and dV; otherwise dQ.
template <typename T, bool KV>
__global__ void __launch_bounds__(256) attn_bwd_tail_sum(const BwdParams p) {
  const int D = p.D, ns = KV ? p.nsplit : p.nsplit_q, nfull = KV ? p.nfull : p.nfull_q;
  const int heads = KV ? p.Hkv : p.H;
  const int64_t nsb = (int64_t)p.B * heads * p.n_blk - nfull;
  const int64_t i4 = (int64_t)block_x() * 256 + thread_x();
  if (i4 >= nsb * 128 * D / 4) return;
  const int64_t row = i4 * 4 / D;
  const int d = (int)(i4 * 4 - row * D);
  const int sbi = (int)(row / 128), rl = (int)(row - (int64_t)sbi * 128);
  int bh, blk;
  if (KV) {
    kv_tile(nfull + sbi, p.B * heads, p.n_blk, false, bh, blk);
  } else {
    FwdParams fp;
    fp.B = p.B; fp.H = p.H; fp.n_qblk = p.n_blk; fp.n_wg = p.B * p.H * p.n_blk;
    wg_tile(nfull + sbi, fp, false, bh, blk);
  }
  const int s = blk * 128 + rl;
  if (s >= (KV ? p.Sk : p.Sq)) return;
  const int b = bh / heads, h = bh - b * heads;
  const float* const src = (KV ? p.part : p.part_q) + row * D + d;
  const int64_t step = nsb * 128 * D;  // one part's floats
  auto sum = [&](const float* base) {
    f32x4 x = *(const f32x4*)base;
    for (int q = 1; q < ns; ++q) x += *(const f32x4*)(base + q * step);
    return x;
  };
  auto put = [&](void* out, int64_t ob, int64_t oh, int64_t os, f32x4 x) {
    u32x2 w;
    w[0] = Elt<T>::pack(x[0], x[1]);
    w[1] = Elt<T>::pack(x[2], x[3]);
    *(u32x2*)((uint16_t*)out + b * ob + h * oh + (int64_t)s * os + d) = w;
  };
  if (KV) {
    put(p.dk, p.dk_b, p.dk_h, p.dk_s, sum(src) * p.scale);
    put(p.dv, p.dv_b, p.dv_h, p.dv_s, sum(src + ns * step));
  } else {
    put(p.dq, p.dq_b, p.dq_h, p.dq_s, sum(src) * p.scale);
  }
}

// Launch the sums of the dK/dV partials (sweeps split nsplit ways) or of the
// dQ partials (nsplit_q ways) that a launch's split sweeps left (errors show
// in the caller's final hipGetLastError).
template <typename T>
void launch_part_sums(const BwdParams& p, bool dkdv, hipStream_t s) {
  PartSum a = {}, b = {};
  if (dkdv) {
    const int64_t rows = (int64_t)p.B * p.Hkv * p.Sk;
    a = PartSum{p.part, p.dk, p.dk_b, p.dk_h, p.dk_s, rows, p.Hkv, p.Sk, p.D, p.nsplit, p.scale};
    b = PartSum{p.part + (int64_t)p.nsplit * rows * p.D, p.dv, p.dv_b, p.dv_h, p.dv_s, rows, p.Hkv, p.Sk, p.D,
                p.nsplit, 1.f};
  } else {
    const int64_t rows = (int64_t)p.B * p.H * p.Sq;
    a = PartSum{p.part_q, p.dq, p.dq_b, p.dq_h, p.dq_s, rows, p.H, p.Sq, p.D, p.nsplit_q, p.scale};
  }
  const int64_t n4 = a.rows * a.D / 4;
  hipLaunchKernelGGL(attn_bwd_part_sum<T>, dim3((unsigned)((n4 + 255) / 256)), dim3(256), 0, s, a, b);
}

// ---- dQ for one block of 128 queries (4 waves x 32 queries), sweeping the
// key tiles (32 rows of K and V) through double-buffered LDS.
template <typename T, int DK, bool CAUSAL, bool MASK>
__global__ void __launch_bounds__(256)
__attribute__((amdgpu_waves_per_eu(DK <= 64 ? (MASK ? 2 : 3) : (DK > 128 || (MASK && CAUSAL)) ? 1 : 2)))
attn_bwd_dq(const BwdParams p) {
  constexpr int BQ = 128, BK = 32;
  constexpr int RS = bwd_lds_stride(DK);
  constexpr int NKS = DK / 16, NDB = DK / 32;
  static_assert(DK % 32 == 0, "head-dim bucket");
  __shared__ __attribute__((aligned(16))) uint16_t lds[2 * 2 * BK * RS];  // [slot][K, V][row][col]
  // D > 64 masked non-causal: the dO operands live in LDS (each lane reads
  // back only what it wrote; no barrier), which leaves room for 2 waves per
  // SIMD instead of 1 (masked backward 473 -> 419 us on bf16
  // [2,16,2048,128]; the causal variant would spill 16 registers and gains
  // nothing, so it keeps its registers and 1 wave)
  constexpr bool DLDS = DK > 64 && DK <= 128 && MASK && !CAUSAL;
  constexpr int RSD = DK + 8;
  __shared__ __attribute__((aligned(16))) uint16_t dpark[DLDS ? BQ * RSD : 8];

  const int tid = thread_x(), wave = tid >> 6, lane = tid & 63, l32 = lane & 31, hh = lane >> 5;
  // split sweeps: (query block, part) pairs as ns virtual blocks per block
  int ns = p.nsplit_q > 1 ? p.nsplit_q : 1;
  int bh, qblk, part, sb = -1;  // sb: index among a split tail's blocks
  if (!CAUSAL && p.nfull_q > 0) {
    // split tail: the first nfull_q workgroups take whole blocks, the rest
    // ns-way parts of the remaining blocks
    const int w = block_x();
    int lb = w;
    part = 0;
    if (w >= p.nfull_q) {
      const int r = w - p.nfull_q;
      lb = p.nfull_q + r / ns;
      part = r - (lb - p.nfull_q) * ns;
      sb = lb - p.nfull_q;
    } else {
      ns = 1;
    }
    FwdParams fp;
    fp.B = p.B; fp.H = p.H; fp.n_qblk = p.n_blk; fp.n_wg = p.B * p.H * p.n_blk;
    wg_tile(lb, fp, false, bh, qblk);
  } else {
    FwdParams fp;
    fp.B = p.B; fp.H = p.H; fp.n_qblk = p.n_blk * ns; fp.n_wg = p.n_wg;
    int vblk;
    wg_tile(block_x(), fp, CAUSAL, bh, vblk);  // causal: longest key sweeps first
    qblk = vblk / ns;
    part = vblk - qblk * ns;
  }
  const int b = bh / p.H, h = bh - b * p.H;
  const int Sq = p.Sq, Sk = p.Sk, D = p.D;
  const int qrow = qblk * BQ + wave * 32 + l32;  // this lane's query

  // B operands held for the whole sweep: 8 head-dim values of this lane's query
  const uint16_t* qg = (const uint16_t*)p.q + b * p.q_b + h * p.q_h;
  const uint16_t* dog = (const uint16_t*)p.dout + b * p.do_b + h * p.do_h;
  u32x4 qf[NKS], dof[DLDS ? 1 : NKS];
  uint16_t* const drow = dpark + (wave * 32 + l32) * RSD + 8 * hh;  // this lane's parked dO
#pragma unroll
  for (int s = 0; s < NKS; ++s) {
    const int d = 16 * s + 8 * hh;
    u32x4 x = {0u, 0u, 0u, 0u}, y = {0u, 0u, 0u, 0u};
    if (qrow < Sq && d < D) {
      x = *(const u32x4*)(qg + (int64_t)qrow * p.q_s + d);
      y = *(const u32x4*)(dog + (int64_t)qrow * p.do_s + d);
    }
    qf[s] = x ^ p.sign;
    if constexpr (DLDS)
      *(u32x4*)(drow + 16 * s) = y;
    else
      dof[s] = y;
  }
  // rows past Sq, and rows that saw no key in the forward (lse = -inf): P = 0
  const float L = qrow < Sq ? p.lse[(int64_t)bh * Sq + qrow] : -INFINITY;
  const float l2 = L > -INFINITY ? L * kLog2e : INFINITY;
  // attention mask rows of this (batch, head); a lane reads its own query row
  const int mkind = MASK ? p.mask_kind : MASK_NONE;
  const int mes = MASK ? mask_bytes(mkind) : 1;
  const __amdgpu_buffer_rsrc_t mrs =
      uniform_rsrc(MASK ? (const void*)((const char*)p.mask + (b * p.m_b + h * p.m_h) * mes) : p.q,
                   MASK ? ((int64_t)(Sq - 1) * p.m_q + (Sk + 7) / 8 * 8) * mes : 0);
  const int mrow_off = MASK ? (int)((int64_t)min(qrow, Sq - 1) * p.m_q * mes) : 0;
  const float dl = qrow < Sq ? p.delta[(int64_t)bh * Sq + qrow] : 0.f;

  const int hk = h / p.group;
  const uint16_t* kg = (const uint16_t*)p.k + b * p.k_b + hk * p.k_h;
  const uint16_t* vg = (const uint16_t*)p.v + b * p.v_b + hk * p.v_h;
  const __amdgpu_buffer_rsrc_t krs = uniform_rsrc(kg, ((int64_t)(Sk - 1) * p.k_s + D) * 2);
  const __amdgpu_buffer_rsrc_t vrs = uniform_rsrc(vg, ((int64_t)(Sk - 1) * p.v_s + D) * 2);
  TileLoader<DK> lk, lv;
  lk.init(tid, p.k_s, D, RS);
  lv.init(tid, p.v_s, D, RS);

  int a_rd[NKS];
  {
    const int r = perm_row(l32);
#pragma unroll
    for (int s = 0; s < NKS; ++s) a_rd[s] = r * RS + 16 * s + 8 * hh;
  }
  const int jj = lane & 15, gg = lane >> 4;
  int t_rd[NDB][2];
#pragma unroll
  for (int db = 0; db < NDB; ++db)
#pragma unroll
    for (int half = 0; half < 2; ++half)
      t_rd[db][half] = (8 * (gg >> 1) + (jj >> 2) + 4 * half) * RS + 32 * db + 16 * (gg & 1) + 4 * (jj & 3);

  f32x16 dqa[NDB];
#pragma unroll
  for (int db = 0; db < NDB; ++db) dqa[db] = (f32x16){};

  const int kend = CAUSAL ? min(Sk, qblk * BQ + BQ) : Sk;  // keys any row of the block sees
  const int nt = (kend + BK - 1) / BK;
  const int wlast = qblk * BQ + wave * 32 + 31;            // this wave's last query
  u32x4 xk[TileLoader<DK>::N], xv[TileLoader<DK>::N];
  auto fetch = [&](int t) {
    lk.load(krs, (int)(t * BK * p.k_s * 2), xk);
    lv.load(vrs, (int)(t * BK * p.v_s * 2), xv);
  };
  auto put = [&](int slot) {
    uint16_t* base = lds + slot * 2 * BK * RS;
    lk.store(base, xk);
    lv.store(base + BK * RS, xv);
  };

  const float c = p.c;
  // this workgroup's key tiles [kt0, kt1) (all of them unless the sweep is split)
  const int kt0 = (int)((int64_t)part * nt / ns), kt1 = (int)((int64_t)(part + 1) * nt / ns);
  if (kt1 > kt0) {
    fetch(kt0);
    put(0);
  }
  lds_barrier();
  for (int t = kt0; t < kt1; ++t) {
    const int slot = (t - kt0) & 1;
    if (t + 1 < kt1) fetch(t + 1);
    const int k0 = t * BK;
    if (!CAUSAL || k0 <= wlast) {  // causal: tiles past this wave's last query add nothing
      const uint16_t* ks = lds + slot * 2 * BK * RS;
      const uint16_t* vs = ks + BK * RS;
      f32x16 s = (f32x16){}, dp = (f32x16){};
#pragma unroll
      for (int st = 0; st < NKS; ++st) s = Elt<T>::mma(*(const u32x4*)(ks + a_rd[st]), qf[st], s);
#pragma unroll
      for (int st = 0; st < NKS; ++st) {
        u32x4 db;
        if constexpr (DLDS)
          db = *(const u32x4*)(drow + 16 * st);
        else
          db = dof[st];
        dp = Elt<T>::mma(*(const u32x4*)(vs + a_rd[st]), db, dp);
      }
      const bool edge = k0 + BK > Sk || (CAUSAL && k0 + BK - 1 > qblk * BQ + wave * 32);
      // mask addends of the lane's 16 keys: two runs of 8 consecutive keys
      // (acc_key), each one 8/16/32-byte read as in the forward
      float madd[16];
      if (MASK) {
#pragma unroll
        for (int run = 0; run < 2; ++run) {
          const int kk = k0 + 16 * run + 8 * hh;
          if (mkind == MASK_BOOL) {
            const u32x2 w = __builtin_bit_cast(u32x2, __builtin_amdgcn_raw_buffer_load_b64(mrs, mrow_off + kk, 0, 0));
#pragma unroll
            for (int i = 0; i < 8; ++i) madd[8 * run + i] = ((w[i >> 2] >> (8 * (i & 3))) & 0xffu) ? 0.f : -INFINITY;
          } else if (mkind == MASK_F32) {
#pragma unroll
            for (int hv = 0; hv < 2; ++hv) {
              const f32x4 a = __builtin_bit_cast(
                  f32x4, __builtin_amdgcn_raw_buffer_load_b128(mrs, mrow_off + 4 * (kk + 4 * hv), 0, 0));
#pragma unroll
              for (int i = 0; i < 4; ++i) madd[8 * run + 4 * hv + i] = a[i] * kLog2e;
            }
          } else {
            const u32x4 w = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(mrs, mrow_off + 2 * kk, 0, 0));
#pragma unroll
            for (int i = 0; i < 4; ++i) {
              const f32x2 a = mkind == MASK_F16 ? Elt<_Float16>::unpack(w[i]) : Elt<__bf16>::unpack(w[i]);
              madd[8 * run + 2 * i] = a[0] * kLog2e;
              madd[8 * run + 2 * i + 1] = a[1] * kLog2e;
            }
          }
        }
      }
      float x[16];
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        x[r] = __builtin_fmaf(s[r], c, -l2);
        if (MASK) x[r] += madd[r];
      }
      // one wave-uniform branch around all 16 checks: per-element branches
      // would be if-converted into selects that every tile pays for
      if (edge) {
        const int lim = CAUSAL ? min(Sk, qrow + 1) : Sk;  // keys below lim count
#pragma unroll
        for (int r = 0; r < 16; ++r)
          if (k0 + acc_key(r, hh) >= lim) x[r] = -INFINITY;
      }
      u32x4 ps[2];
#pragma unroll
      for (int ks2 = 0; ks2 < 2; ++ks2)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          float pv[2];
#pragma unroll
          for (int u = 0; u < 2; ++u) {
            const int r = 8 * ks2 + 2 * e + u;
            pv[u] = fast_exp2(x[r]) * (dp[r] - dl);
          }
          ps[ks2][e] = Elt<T>::pack(pv[0], pv[1]);
        }
      // dQ^T += K^T dS^T (16 keys per k-step)
#pragma unroll
      for (int ks2 = 0; ks2 < 2; ++ks2)
#pragma unroll
        for (int db = 0; db < NDB; ++db)
          dqa[db] = Elt<T>::mma(tr_frag(ks + 16 * ks2 * RS, t_rd[db][0], t_rd[db][1]), ps[ks2], dqa[db]);
    }
    if (t + 1 < kt1) put(slot ^ 1);
    lds_barrier();
  }

  if (ns > 1 && sb >= 0) {  // split tail: block-indexed partial rows, unscaled
    const int64_t nsb = (int64_t)p.B * p.H * p.n_blk - p.nfull_q;
    store_rows_f32<NDB>(p.part_q + ((int64_t)part * nsb + sb) * BQ * D, qrow - qblk * BQ, Sq - qblk * BQ, D, hh,
                        dqa);
    return;
  }
  if (ns > 1) {  // this part's partial rows, unscaled
    store_rows_f32<NDB>(p.part_q + ((int64_t)part * p.B * p.H + bh) * Sq * D, qrow, Sq, D, hh, dqa);
    return;
  }
  uint16_t* dqg = (uint16_t*)p.dq + b * p.dq_b + h * p.dq_h;
  store_rows<T, NDB>(dqg, p.dq_s, qrow, Sq, D, hh, dqa, p.scale);
}

}  // namespace cmpext3
