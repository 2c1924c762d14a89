// Decode-step attention forward for fp16 / bf16 on gfx950: few query rows per
// K/V head (a decode step, or a short speculative block), a long key sweep.
//
// Such a launch moves almost nothing but K and V (B * H_kv heads of Sk rows
// each, read once), so it is bound by how many bytes the chip keeps in flight
// from HBM, not by arithmetic.  The prefill kernels stream K/V through a ring
// shared by a workgroup's waves, with a barrier per tile and one or two tiles
// ahead; here every wave streams its own key tiles, so nothing waits for
// another wave until the end:
//
//  * Problem: one "unit" per (batch, K/V head) whose R <= 16 rows are the
//    query rows of that head (the query heads of a group packed as rows:
//    FwdParams::pack_sq).  A unit's keys are cut into `parts` ranges, one per
//    workgroup, and a workgroup's 16-key tiles are dealt to its four waves in
//    turn (wave w: tiles w, w + 4, ...), so the four stream adjacent memory.
//  * Each wave owns a ring of NS stages in LDS (K tile then V tile, 16 rows
//    each) filled by buffer_load ... lds (no staging registers): it issues the
//    loads of tile j + NS as soon as it has read tile j, and waits for a tile
//    with s_waitcnt vmcnt, never with a barrier.
//  * Scores S^T = K Q^T with v_mfma_f32_16x16x32 (a lane holds 4 keys of one
//    query row), exact online softmax in the exp2 domain (the running max is
//    raised only when a tile exceeds it: a wave-uniform branch), P^T straight
//    from the score registers into v_mfma_f32_16x16x16 with V^T read by
//    ds_read_b64_tr_b16: O^T = V^T P^T, a lane holding one row's 4 columns of
//    each 16-column block.
//  * End: the four waves' (O, m, l) meet in LDS and are merged; with one part
//    the workgroup writes the output, otherwise it leaves its merged state in
//    the exchange space (the caller's workspace or the fixed scratch) and
//    counts itself in; the last part of a unit merges every part in part
//    order and puts the unit's counter back to zero.  Nobody waits for
//    another workgroup.
//
// Reference algorithm: src/cuda/fp16_flash_attention_hfma2.cu:72-243 (exp2
// online softmax with fp32 running max/sum and output, one final 1/l), the
// split-KV decode of 002-cmp-flash-attention.patch:473-492 (partial results
// combined with their (m, l)).
#include <stdio.h>

#include "attn_common.h"

namespace cmpext3 {

namespace {

typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x2d __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2d __attribute__((ext_vector_type(2)));
typedef short i16x4d __attribute__((ext_vector_type(4)));
typedef float f32x2d __attribute__((ext_vector_type(2)));

template <typename T> struct Dec;

template <> struct Dec<_Float16> {
  static __device__ __forceinline__ f32x4 qk(u32x4 a, u32x4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c,
                                                  0, 0, 0);
  }
  static __device__ __forceinline__ f32x4 pv(u32x2 a, u32x2 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x16f16(__builtin_bit_cast(f16x4, a), __builtin_bit_cast(f16x4, b), c,
                                                 0, 0, 0);
  }
  static __device__ __forceinline__ uint32_t pack(float a, float b) {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2d){a, b}, f16x2d));
  }
  static __device__ __forceinline__ float sum2(uint32_t w, float acc) {
    return __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2d, w), (f16x2d){1.0f16, 1.0f16}, acc, false);
  }
};

template <> struct Dec<__bf16> {
  static __device__ __forceinline__ f32x4 qk(u32x4 a, u32x4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b),
                                                   c, 0, 0, 0);
  }
  static __device__ __forceinline__ f32x4 pv(u32x2 a, u32x2 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(__builtin_bit_cast(i16x4d, a), __builtin_bit_cast(i16x4d, b),
                                                     c, 0, 0, 0);
  }
  static __device__ __forceinline__ uint32_t pack(float a, float b) {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2d){a, b}, bf16x2d));
  }
  static __device__ __forceinline__ float sum2(uint32_t w, float acc) {
    const bf16x2d one = {(__bf16)1.0f, (__bf16)1.0f};
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2d, w), one, acc, false);
  }
};

constexpr int kDecNw = 4;           // waves per workgroup
constexpr int kDecRows = 16;        // query rows per unit at most
constexpr int kDecBk = 16;          // keys per tile
constexpr int kDecMinTiles = 4;     // tiles per wave at least, when keys are split
constexpr int kDecMaxParts = 128;   // key ranges per unit at most
constexpr int kDecMergeLoads = 8;   // exchange loads of one merging thread in flight together
constexpr int kDecLds = 160 * 1024; // LDS of one CU

// Ring stages per wave: as deep as 128 KB of LDS per workgroup allows, at
// most 4 (measured on MI355X: deeper rings, up to the CU's 160 KB, were 9-13%
// slower at D = 160 and 192: more requests in flight than HBM serves well).
constexpr int dec_stages(int dk) {
  return 128 * 1024 / (kDecNw * 2 * kDecBk * dk * 2) < 4 ? 128 * 1024 / (kDecNw * 2 * kDecBk * dk * 2) : 4;
}
constexpr int dec_lds_bytes(int dk) { return kDecNw * dec_stages(dk) * 2 * kDecBk * dk * 2; }

// Physical 16-byte chunk of logical chunk c in LDS row r (nc chunks a row):
// XOR with f(r) = 2 (r mod 4) + (r / 4 mod 2) inside every whole group of 8
// chunks; chunks of a last, partial group stay in place.  The K fragment
// reads (8 lanes a pass: rows 0-7 or 8-15, one chunk) and the transposed V
// reads (16 lanes a pass: rows 4g..4g+3, two neighbouring chunks) then touch
// distinct 16-byte bank groups where the row length is a multiple of 128
// bytes.  An involution: the same function maps back.
__device__ __forceinline__ int dec_swz(int r, int c, int nc) {
  const int f = ((r & 3) << 1) | ((r >> 2) & 1);
  return c < (nc & ~7) ? (c ^ f) : c;
}

struct DecArgs {
  int rows;    // query rows per unit (R <= 16)
  int nt;      // 16-key tiles per unit
  int parts;   // workgroups per unit (key ranges)
  f32x4* ws;   // exchange: [unit][part][row] (DK / 4 + 1) float4: O, then (m, l, 0, 0)
  int* cnt;    // one counter per unit, then (two-level merge) one per group of
               // each unit from cnt + gbase; zero between launches
  int gsize;   // parts per merge group (>= parts: one-level merge)
  int gbase;   // index of the first group counter
};

__device__ __forceinline__ float shfl_xor_f(float x, int m) { return __shfl_xor(x, m); }

// Offset (elements) of query row r of a unit: packed rows walk the group's
// query heads (q_g) and positions (q_s); otherwise rows are positions.
__device__ __forceinline__ int64_t dec_row(int r, int pack_sq, int64_t g_str, int64_t s_str) {
  if (pack_sq > 0) {
    const int h = r / pack_sq;
    return (int64_t)h * g_str + (int64_t)(r - h * pack_sq) * s_str;
  }
  return (int64_t)r * s_str;
}

template <typename T, int DK>
__global__ __launch_bounds__(kDecNw * 64, 1) void attn_fwd_decode16(FwdParams p, DecArgs a) {
  constexpr int NS = dec_stages(DK);
  constexpr int RB = DK * 2;            // bytes of a K/V row in LDS
  constexpr int NC = DK / 8;            // 16-byte chunks per row
  constexpr int BLK = kDecBk * RB;      // bytes of one 16-row block
  constexpr int IB = BLK / 1024;        // DMA instructions per block (64 lanes x 16 bytes)
  constexpr int STAGE = 2 * BLK;
  constexpr int KS = DK / 32;           // score k-steps
  constexpr int NDB = DK / 16;          // 16-column output blocks
  constexpr int DQ = DK / 4;            // float4 vectors of an output row
  static_assert(DK % 32 == 0 && DK >= 64 && DK <= 256, "head dim");
  static_assert(BLK % 1024 == 0, "a block is whole DMA instructions");
  static_assert(2 * IB * (NS - 1) <= 63, "vmcnt range");
  constexpr int MOS = DK + 4;           // row stride (floats) of the waves' merge rows
  static_assert(kDecNw * kDecRows * MOS * 4 + 2 * kDecNw * kDecRows * 4 + 16 <= kDecNw * NS * STAGE,
                "the workgroup's merge fits in the ring's LDS");
  static_assert(2 * kDecRows * kDecMaxParts * 4 + 2 * kDecRows * 4 + 16 + kDecNw * 64 * 16 <= kDecNw * NS * STAGE,
                "the parts' merge fits in the ring's LDS");
  __shared__ __attribute__((aligned(16))) unsigned char lds[kDecNw * NS * STAGE];

  const int tid = thread_x(), lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wg = block_x();
  const int unit = wg / a.parts, part = wg - unit * a.parts;
  const int b = unit / p.H, hk = unit - b * p.H;
  const int R = a.rows, Sk = p.Sk, D = p.D;
  const int t0 = (int)((int64_t)part * a.nt / a.parts);
  const int t1 = (int)((int64_t)(part + 1) * a.nt / a.parts);
  const int mine = t1 - t0 > wave ? (t1 - t0 - wave + kDecNw - 1) / kDecNw : 0;  // tiles of this wave

  const uint16_t* qg = (const uint16_t*)p.q + b * p.q_b + hk * p.q_h;
  const uint16_t* kg = (const uint16_t*)p.k + b * p.k_b + (int64_t)(hk / p.kv_group) * p.k_h;
  const uint16_t* vg = (const uint16_t*)p.v + b * p.v_b + (int64_t)(hk / p.kv_group) * p.v_h;
  uint16_t* og = (uint16_t*)p.o + b * p.o_b + hk * p.o_h;

  const int c = lane & 15, g = lane >> 4;

  // Q^T fragments (B operand of the score MFMA): row c, columns 32 ks + 8 g ..
  u32x4 qf[KS];
  {
    const bool live = c < R;
    const uint16_t* qrow = qg + (live ? dec_row(c, p.pack_sq, p.q_g, p.q_s) : 0);
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      u32x4 x = live ? *(const u32x4*)(qrow + 32 * ks + 8 * g) : (u32x4){0u, 0u, 0u, 0u};
      x ^= (u32x4){p.q_sign, p.q_sign, p.q_sign, p.q_sign};
      qf[ks] = x;
    }
  }

  // DMA: instruction i of a block writes LDS bytes [1024 i, 1024 i + 1024);
  // lane l's 16 bytes land at 1024 i + 16 l, i.e. row r, physical chunk pc,
  // which holds logical chunk dec_swz(r, pc) of key row r.
  const int ks_b = (int)p.k_s * 2, vs_b = (int)p.v_s * 2;
  int kdo[IB], vdo[IB];
#pragma unroll
  for (int i = 0; i < IB; ++i) {
    const int pos = 1024 * i + 16 * lane;
    const int r = pos / RB, pc = (pos - r * RB) / 16;
    const int lc = dec_swz(r, pc, NC);
    kdo[i] = r * ks_b + 16 * lc;
    vdo[i] = r * vs_b + 16 * lc;
  }
  // K fragment reads (A operand): key row c, logical chunk 4 ks + g
  int kro[KS];
#pragma unroll
  for (int ks = 0; ks < KS; ++ks) kro[ks] = c * RB + 16 * dec_swz(c, 4 * ks + g, NC);
  // transposed V reads (A operand of O^T = V^T P^T): 16 lanes of group g read
  // rows 4g..4g+3 x columns 16 db .. 16 db + 15, lane jj the 4 columns
  // 16 db + 4 (jj & 3) of row 4 g + jj / 4, and lane jj receives column
  // 16 db + jj of the four rows
  int vro[NDB];
#pragma unroll
  for (int db = 0; db < NDB; ++db) {
    const int r = 4 * g + (c >> 2), col = 16 * db + 4 * (c & 3);
    vro[db] = r * RB + 16 * dec_swz(r, col >> 3, NC) + 2 * (col & 7);
  }

  typedef __attribute__((address_space(3))) unsigned char lds_u8;
  const uint32_t lds0 = (uint32_t)(uintptr_t)(lds_u8*)lds;
  const uint32_t ring = lds0 + (uint32_t)(wave * NS * STAGE);
  const u32x4 krw = uniform_rsrc_words(kg, ((int64_t)(Sk - 1) * p.k_s + D) * 2);
  const u32x4 vrw = uniform_rsrc_words(vg, ((int64_t)(Sk - 1) * p.v_s + D) * 2);
  // this wave's tile j into stage j % NS (rows past Sk read zeros)
  auto issue = [&](int j) {
    const int key0 = (t0 + wave + kDecNw * j) * kDecBk;
    const uint32_t st = ring + (uint32_t)((j % NS) * STAGE);
    const int sk = key0 * ks_b, sv = key0 * vs_b;
#pragma unroll
    for (int i = 0; i < IB; ++i) lds_dma16(krw, st + 1024 * i, kdo[i], sk);
#pragma unroll
    for (int i = 0; i < IB; ++i) lds_dma16(vrw, st + BLK + 1024 * i, vdo[i], sv);
  };

  f32x4 oacc[NDB];
#pragma unroll
  for (int db = 0; db < NDB; ++db) oacc[db] = (f32x4){0.f, 0.f, 0.f, 0.f};
  float m_run = -INFINITY, l_run = 0.f;
  const float cmul = p.c;

#pragma unroll
  for (int j = 0; j < NS; ++j)
    if (j < mine) issue(j);

  for (int j = 0; j < mine; ++j) {
    // tile j has landed once at most (tiles still in flight behind it) x
    // (instructions per tile) loads are outstanding
    const int behind = min(NS - 1, mine - 1 - j);
    if (behind >= 3) wait_vmcnt<6 * IB>();
    else if (behind == 2) wait_vmcnt<4 * IB>();
    else if (behind == 1) wait_vmcnt<2 * IB>();
    else wait_vmcnt<0>();
    const unsigned char* st = lds + (wave * NS + j % NS) * STAGE;
    const int key0 = (t0 + wave + kDecNw * j) * kDecBk;

    f32x4 s = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) s = Dec<T>::qk(*(const u32x4*)(st + kro[ks]), qf[ks], s);

    float x[4];
    if (key0 + kDecBk <= Sk) {
#pragma unroll
      for (int e = 0; e < 4; ++e) x[e] = s[e] * cmul;
    } else {
#pragma unroll
      for (int e = 0; e < 4; ++e) x[e] = key0 + 4 * g + e < Sk ? s[e] * cmul : -INFINITY;
    }
    float mt = fmaxf(fmaxf(x[0], x[1]), fmaxf(x[2], x[3]));
    mt = fmaxf(mt, shfl_xor_f(mt, 16));
    mt = fmaxf(mt, shfl_xor_f(mt, 32));
    if (__builtin_amdgcn_ballot_w64(mt > m_run)) {  // some row's maximum rises
      const float m_new = fmaxf(m_run, mt);
      const float alpha = fast_exp2(m_run - m_new);  // 0 on the first tile (m_run = -inf)
      m_run = m_new;
      l_run *= alpha;
#pragma unroll
      for (int db = 0; db < NDB; ++db) oacc[db] *= alpha;
    }
    u32x2 pb;
    pb[0] = Dec<T>::pack(fast_exp2(x[0] - m_run), fast_exp2(x[1] - m_run));
    pb[1] = Dec<T>::pack(fast_exp2(x[2] - m_run), fast_exp2(x[3] - m_run));
    l_run = Dec<T>::sum2(pb[1], Dec<T>::sum2(pb[0], l_run));  // the rounded P the PV MFMA takes

    const uint16_t* vs = (const uint16_t*)(st + BLK);
#pragma unroll
    for (int db = 0; db < NDB; ++db) {
      typedef __attribute__((address_space(3))) i16x4d lds_i16x4;
      const i16x4d v = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)((const unsigned char*)vs + vro[db]));
      oacc[db] = Dec<T>::pv(__builtin_bit_cast(u32x2, v), pb, oacc[db]);
    }
    if (j + NS < mine) {
      // this stage's LDS reads have returned before its next tile's loads go out
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
      issue(j + NS);
    }
  }

  // ---- the four waves' states meet in LDS: [wave][row][DK] O, then m, l
  float lrow = l_run + shfl_xor_f(l_run, 16);
  lrow += shfl_xor_f(lrow, 32);
  wait_vmcnt<0>();
  lds_barrier();  // every wave is done with its ring
  // (rows 16 bytes apart mod 128: the 16-byte writes of 8 rows per LDS pass
  // land on distinct banks)
  float* mo = (float*)lds;
  float* mm = mo + kDecNw * kDecRows * MOS;
  float* ml = mm + kDecNw * kDecRows;
#pragma unroll
  for (int db = 0; db < NDB; ++db) *(f32x4*)(mo + (wave * kDecRows + c) * MOS + 16 * db + 4 * g) = oacc[db];
  if (g == 0) {
    mm[wave * kDecRows + c] = m_run;
    ml[wave * kDecRows + c] = lrow;
  }
  lds_barrier();

  const int nparts = a.parts;
  const int nu = R * DQ;  // (row, 4 columns) units of the output
  const __amdgpu_buffer_rsrc_t wsr =
      uniform_rsrc(nparts > 1 ? (const void*)a.ws : (const void*)mo,
                   nparts > 1 ? (int64_t)(unit + 1) * nparts * R * (DQ + 1) * 16 : 16);
  auto slot = [&](int q, int r, int k) { return (((unit * nparts + q) * R + r) * (DQ + 1) + k) * 16; };
  auto store_out = [&](int r, int k, f32x4 o, float inv) {
    u32x2 w;
    w[0] = Dec<T>::pack(o[0] * inv, o[1] * inv);
    w[1] = Dec<T>::pack(o[2] * inv, o[3] * inv);
    *(u32x2*)(og + dec_row(r, p.pack_sq, p.o_g, p.o_s) + 4 * k) = w;
  };
  for (int u = tid; u < nu; u += kDecNw * 64) {
    const int r = u / DQ, k = u - r * DQ;
    float mw[kDecNw], mx = -INFINITY;
#pragma unroll
    for (int w = 0; w < kDecNw; ++w) {
      mw[w] = mm[w * kDecRows + r];
      mx = fmaxf(mx, mw[w]);
    }
    f32x4 o = {0.f, 0.f, 0.f, 0.f};
    float l = 0.f;
#pragma unroll
    for (int w = 0; w < kDecNw; ++w) {
      const float f = mw[w] == -INFINITY ? 0.f : fast_exp2(mw[w] - mx);  // a wave without tiles: 0
      l = __builtin_fmaf(ml[w * kDecRows + r], f, l);
      o += *(const f32x4*)(mo + (w * kDecRows + r) * MOS + 4 * k) * f;
    }
    if (nparts == 1) {
      store_out(r, k, o, 1.f / l);
    } else {
      // device-scope (aux 16 = sc1) stores, coherent across the XCDs' L2s
      __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, o), wsr, slot(part, r, k), 0, 16);
      if (k == 0)
        __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, ((f32x4){mx, l, 0.f, 0.f})), wsr,
                                               slot(part, r, DQ), 0, 16);
    }
  }
  if (nparts == 1) return;

  // ---- key split: count in; the last arriver merges.  One level: the last
  // part of the unit merges every part.  Two levels (deep splits, a.gsize <
  // nparts): the last part of each group of a.gsize consecutive parts merges
  // the group into the group's first slot, unnormalised, and counts the group
  // in; the last group merges the groups.  Counters go back to zero.
  int* const flag = (int*)(ml + kDecNw * kDecRows);
  const int gs = a.gsize, ng = (nparts + gs - 1) / gs;
  auto count_in = [&](int* ctr, int n) {
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    lds_barrier();  // every wave's stores are done (and its LDS reads)
    if (tid == 0) {
      const int old = __hip_atomic_fetch_add(ctr, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      if (old == n - 1) __hip_atomic_store(ctr, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      *flag = old == n - 1;
    }
    lds_barrier();
    const bool last = __builtin_amdgcn_readfirstlane(*flag) != 0;
    asm volatile("" ::: "memory");  // the exchange loads stay after the count
    if (last) lds_barrier();        // every wave has read the flag before its LDS is reused
    return last;
  };
  auto ld = [&](int off) {
    return __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(wsr, off, 0, 16));
  };
  // Merge the n entries q0, q0 + qs, ... of this unit's exchange.  The merge
  // is on the launch's tail, so it is laid out for few dependent memory round
  // trips: (1) every entry's (m, l) of every row in one load per thread, then
  // per row (one wave each) the weight of each entry, exp2(m_q - max m),
  // divided by the weighted row-sum total for the output; (2) every thread
  // loads all of its share of the partial outputs at once: the entries of an
  // output vector are spread over S thread groups whose sums meet in LDS.
  // `fin` writes the output; otherwise the unnormalised (O, max m, total)
  // goes to entry q0.  Fixed assignment and summation order: the same result
  // whichever part merges.
  auto merge = [&](int q0, int qs, int n, bool fin) {
    float* const wq = (float*)lds;  // [row][entry] offsets, then weights
    float* const lq = wq + R * n;   // [row][entry] row sums
    float* const rt = lq + R * n;   // [row] (max m, total) of a group merge
    for (int i = tid; i < R * n; i += kDecNw * 64) {
      const int r = i / n, j = i - r * n;
      const f32x4 e = ld(slot(q0 + j * qs, r, DQ));
      wq[i] = e[0];
      lq[i] = e[1];
    }
    lds_barrier();
    for (int r = wave; r < R; r += kDecNw) {
      float* const wr = wq + r * n;
      const float* const lr = lq + r * n;
      float mx = -INFINITY;
      for (int j = lane; j < n; j += 64) mx = fmaxf(mx, wr[j]);  // every part has keys: finite
#pragma unroll
      for (int m = 32; m >= 1; m >>= 1) mx = fmaxf(mx, shfl_xor_f(mx, m));
      float L = 0.f;
      for (int j = lane; j < n; j += 64) L = __builtin_fmaf(lr[j], fast_exp2(wr[j] - mx), L);
#pragma unroll
      for (int m = 32; m >= 1; m >>= 1) L += shfl_xor_f(L, m);
      const float inv = fin ? 1.f / L : 1.f;
      for (int j = lane; j < n; j += 64) wr[j] = fast_exp2(wr[j] - mx) * inv;  // this lane's own entries
      if (!fin && lane == 0) {
        rt[2 * r] = mx;
        rt[2 * r + 1] = L;
      }
    }
    lds_barrier();
    constexpr int NT = kDecNw * 64;
    constexpr int CH = kDecMergeLoads;
    const int S = nu >= NT ? 1 : NT / nu;
    f32x4* const acc = (f32x4*)(lds + ((2 * R * n * 4 + 2 * R * 4 + 15) & ~15));  // [S][nu] partial sums
    auto put = [&](int r, int k, f32x4 o) {
      if (fin) {
        store_out(r, k, o, 1.f);
      } else {
        __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, o), wsr, slot(q0, r, k), 0, 16);
        if (k == 0)
          __builtin_amdgcn_raw_buffer_store_b128(
              __builtin_bit_cast(u32x4, ((f32x4){rt[2 * r], rt[2 * r + 1], 0.f, 0.f})), wsr, slot(q0, r, DQ), 0,
              16);
      }
    };
    for (int u0 = 0; u0 < nu; u0 += NT / S) {
      const int t = tid % (NT / S), sg = tid / (NT / S), u = u0 + t;
      f32x4 o = {0.f, 0.f, 0.f, 0.f};
      if (u < nu && sg < S) {
        const int r = u / DQ, k = u - r * DQ;
        const float* const wr = wq + r * n;
        for (int j0 = sg; j0 < n; j0 += CH * S) {
          f32x4 x[CH];
#pragma unroll
          for (int i = 0; i < CH; ++i) {
            const int j = j0 + i * S;
            x[i] = j < n ? ld(slot(q0 + j * qs, r, k)) : (f32x4){0.f, 0.f, 0.f, 0.f};
          }
#pragma unroll
          for (int i = 0; i < CH; ++i) {
            const int j = j0 + i * S;
            if (j < n) o += x[i] * wr[j];
          }
        }
        if (S == 1) put(r, k, o);
      }
      if (S > 1) {
        if (sg < S && u < nu) acc[sg * nu + u] = o;  // S > 1: nu < NT, one pass (u0 = 0)
        lds_barrier();
        if (tid < nu) {
          f32x4 sum = acc[tid];
          for (int g2 = 1; g2 < S; ++g2) sum += acc[g2 * nu + tid];
          put(tid / DQ, tid - tid / DQ * DQ, sum);
        }
      }
    }
  };
  if (gs >= nparts) {
    if (count_in(a.cnt + unit, nparts)) merge(0, 1, nparts, true);
    return;
  }
  const int grp = part / gs, g0 = grp * gs;
  const int gn = nparts - g0 < gs ? nparts - g0 : gs;
  if (!count_in(a.cnt + a.gbase + unit * ng + grp, gn)) return;
  merge(g0, 1, gn, false);
  if (count_in(a.cnt + unit, ng)) merge(0, gs, ng, true);
}

template <typename T, int DK>
hipError_t launch_dk(const FwdParams& p, const DecArgs& a, int units, hipStream_t s) {
  hipLaunchKernelGGL((attn_fwd_decode16<T, DK>), dim3(units * a.parts), dim3(kDecNw * 64), 0, s, p, a);
  return hipGetLastError();
}

template <typename T>
hipError_t launch_t(const FwdParams& p, const DecArgs& a, int units, hipStream_t s) {
  switch (p.D) {
    case 64: return launch_dk<T, 64>(p, a, units, s);
    case 96: return launch_dk<T, 96>(p, a, units, s);
    case 128: return launch_dk<T, 128>(p, a, units, s);
    case 160: return launch_dk<T, 160>(p, a, units, s);
    case 192: return launch_dk<T, 192>(p, a, units, s);
    case 224: return launch_dk<T, 224>(p, a, units, s);
    case 256: return launch_dk<T, 256>(p, a, units, s);
  }
  return hipErrorInvalidValue;
}

}  // namespace

bool packs_query_heads(const FwdParams& p, bool causal);
void pack_query_heads(FwdParams& p);

// Head dims of this kernel: whole 32-column score steps, 64 to 256.
static bool decode16_dim(int D) { return D % 32 == 0 && D >= 64 && D <= 256; }

// True when a launch is a decode shape this kernel takes: non-causal,
// unmasked inference with whole aligned 16-byte chunks, at most 16 query rows
// per K/V head once grouped query heads are packed, key rows that do not
// overlap (rows past Sk then lie past the buffer and read zeros) and every
// tile addressable with 32-bit buffer offsets.  Up to D = 128 the pipelined
// kernel's decode path is as fast while the units (batch x K/V heads) fill
// half the CUs or more (within 2-4% either way on MI355X); below that its key
// split cuts deeper and this kernel's merge wins (1.4-2x at 8 units).
bool decode16_applies(const FwdParams& p, bool causal) {
  if (causal || p.mask_kind != MASK_NONE || p.lse || p.elem_rows || !decode16_dim(p.D)) return false;
  const bool packs = packs_query_heads(p, causal);
  const int64_t rows = packs ? (int64_t)p.kv_group * p.Sq : p.Sq;
  if (rows > kDecRows) return false;
  const int64_t units = (int64_t)p.B * (packs ? p.H / p.kv_group : p.H);
  if (p.D <= 128 && 2 * units >= device_cus()) return false;
  const int64_t ks = p.Sk > 1 ? p.k_s : p.D, vs = p.Sk > 1 ? p.v_s : p.D;
  if (ks < p.D || vs < p.D) return false;
  return (int64_t)(p.Sk + kDecBk) * (ks > vs ? ks : vs) * 2 < (int64_t)INT32_MAX;
}

namespace {

int dec_stages_of(int D) {
  switch (D) {
    case 64: return dec_stages(64);
    case 96: return dec_stages(96);
    case 128: return dec_stages(128);
    case 160: return dec_stages(160);
    case 192: return dec_stages(192);
    case 224: return dec_stages(224);
  }
  return dec_stages(256);
}

int dec_lds(int D) { return kDecNw * dec_stages_of(D) * 2 * kDecBk * D * 2; }

// Key ranges per unit: enough workgroups to fill every CU slot the LDS
// allows, each wave keeping at least kDecMinTiles tiles.
int dec_parts(int units, int nt, int D, int cus) {
  const int slots = cus * (kDecLds / dec_lds(D));
  if (units >= slots) return 1;
  int parts = (slots + units - 1) / units;
  const int cap = nt / (kDecNw * kDecMinTiles) < kDecMaxParts ? nt / (kDecNw * kDecMinTiles) : kDecMaxParts;
  if (parts > cap) parts = cap;
  return parts >= 2 ? parts : 1;
}

// Parts per merge group.  The merging workgroup loads kDecMergeLoads partial
// vectors per thread at a time; a split whose one-level merge needs eight or
// more such batches per thread (deep splits of many rows: 64 parts of 8 rows
// at D = 256 take 16) merges in two levels of about sqrt(parts) entries each
// (on MI355X, [1,32/4,1,65536,256]: the one-level merge took 16.6 us of a
// 60.9 us launch).  Otherwise one level (returns parts).
int dec_group(int parts, int rows, int D) {
  const int nt = kDecNw * 64, nu = rows * (D / 4);
  const int S = nu >= nt ? 1 : nt / nu;
  const int passes = S == 1 ? (nu + nt - 1) / nt : 1;  // output vectors per thread
  const int batches = passes * ((parts + kDecMergeLoads * S - 1) / (kDecMergeLoads * S));
  if (batches < 8) return parts;
  int g = 1;
  while (g * g < parts) ++g;
  return g;
}

}  // namespace

hipError_t launch_decode16(const FwdParams& p0, bool bf16, hipStream_t s) {
  FwdParams p = p0;
  if (packs_query_heads(p, false)) pack_query_heads(p);
  if (p.Sk == 1) p.k_s = p.v_s = p.D;  // one row: rows past it must lie past the buffer
  const int units = p.B * p.H;
  if (units == 0) return hipSuccess;
  DecArgs a = {p.Sq, (p.Sk + kDecBk - 1) / kDecBk, 1, nullptr, nullptr, 1, units};
  const int parts = dec_parts(units, a.nt, p.D, device_cus());
  if (parts >= 2) {
    const size_t part_bytes = (size_t)units * a.rows * (p.D / 4 + 1) * sizeof(f32x4);
    // counters for the two-level merge of the deepest plan (fewer parts need fewer)
    const int gs = dec_group(parts, a.rows, p.D);
    const int ncnt = units * (1 + (parts + gs - 1) / gs);
    const int fit = bind_exchange(p, parts, part_bytes, ncnt, &a.ws, &a.cnt);
    if (fit >= 2) {
      a.parts = fit;
      a.gsize = dec_group(fit, a.rows, p.D);
    }
  } else if (p.dry) {
    *p.dry = SplitInfo{0, 1};
  }
  if (p.dry) return hipSuccess;
  return bf16 ? launch_t<__bf16>(p, a, units, s) : launch_t<_Float16>(p, a, units, s);
}

void describe_decode16(int D, int B, int H, int Sq, int Sk, char* buf, int len) {
  const int nt = (Sk + kDecBk - 1) / kDecBk;
  const int parts = dec_parts(B * H, nt, D, device_cus());
  char split[64] = "";
  if (parts >= 2) {
    const int gs = dec_group(parts, Sq, D);
    const int n = snprintf(split, sizeof split, " key-split: %d x %d parts", B * H, parts);
    if (gs < parts) snprintf(split + n, sizeof split - n, ", merged in groups of %d", gs);
  }
  snprintf(buf, len,
           "decode16 16x16 S^T-form: DK=%d rows=%d waves=%d BK=%d, a %d-stage LDS DMA ring per wave, "
           "workgroups/CU=%d%s",
           D, Sq, kDecNw, kDecBk, dec_stages_of(D), kDecLds / dec_lds(D), split);
}

}  // namespace cmpext3
