// Backward pass of the fused attention for fp32 on gfx950 fp32 MFMA
// (v_mfma_f32_16x16x4f32: exact fp32 products, fp32 accumulation), head-dim
// buckets 32, 40, 64, 96, 128, 192 and 256 (columns past D are zero in every
// operand and never stored).
//
// The same gradients as the fp16/bf16 backward (attn_bwd16.h), with
// P = exp2(S * c - lse * log2 e) rebuilt from the forward's row log-sum-exp:
//   Delta_i = sum_d dO_id O_id                     (attn_bwd32_delta)
//   dV = P^T dO,  dK = scale * dS^T Q              (attn_bwd32_dkdv, per 64 keys)
//   dQ = scale * dS K                              (attn_bwd32_dq, per 64 queries)
//   with dP = dO V^T and dS = P * (dP - Delta).
// Each gradient row is written by exactly one workgroup (no atomics), so the
// results are bit-identical from run to run.
//
// Layout of a 16x16x4 MFMA: A lane (l16, g) = A[l16][g], B lane (l16, g) =
// B[g][l16], C lane (l16, g) = C[4g + i][l16], i = 0..3.
//  * dK/dV (lane = key l16 of the wave's 16): S = Q K^T and dP = dO V^T take
//    their B operand (K, V of the lane's key: one float per k-step) from
//    registers and their A operand (query rows) from the LDS tile, so a lane
//    holds S[4 consecutive queries][its key].  Element r of P and dS is then
//    exactly the B operand of dV^T += dO^T P and dK^T += Q^T dS at the k-step
//    whose A operand holds query 4g + r: dO^T[d][4g + r] read from the LDS
//    tile along d.  The accumulators hold dV^T[4 consecutive d][key].
//  * dQ (lane = query): S^T = K Q^T and dP^T = V dO^T (Q, dO in registers),
//    and dQ^T += K^T dS^T the same way.
// LDS tiles: [rows][RS] fp32 with RS = 4 * odd floats, and the two 8-byte
// halves of every 16-byte chunk swapped in rows with bit 3 set, so that both
// reads are free of bank conflicts: 16 rows x 4 consecutive columns (rows l
// and l + 8 fall on the same banks, the swap moves row l + 8 to the other
// lane-group pair) and 4 rows 4 apart x 16 consecutive columns (4 * RS is 16
// banks mod 32).
//
// Reference: none.  The reference is forward-only: its patch hands every call
// with live autograd to stock torch (cmpext3/__init__.py:115-125).
#include "attn_bwd16.h"

namespace cmpext3 {

namespace {

__device__ __forceinline__ f32x4 mma4(float a, float b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

// LDS row stride (floats) of a tile with `cols` columns: 4 * odd
constexpr int rs32(int cols) { return (cols / 4) % 2 == 0 ? cols + 4 : cols; }

// Lane bases of the two tile reads (the 8-byte halves of each 16-byte chunk
// trade places in rows with bit 3 set), to which whole 16-row blocks, 4-column
// k-steps and 16-column blocks add constant offsets:
//  * rows l16 (+ 16 j), columns 4 s + g: l16 * RS + (g ^ swap(l16)) + 16 j RS + 4 s
//  * rows 4 g + r (+ 16 j), columns l16 (+ 16 db): (4 g + r) RS + (l16 ^ swap(4 g + r)) + 16 j RS + 16 db
__device__ __forceinline__ int sbase(int l16, int g, int RS) { return l16 * RS + (g ^ ((l16 >> 2) & 2)); }
__device__ __forceinline__ int tbase(int l16, int g, int r, int RS) { return (4 * g + r) * RS + (l16 ^ (g & 2)); }

// ROWS x CW-column fp32 tile of a [rows, D] matrix into registers and then
// into LDS: 16-byte chunks spread over the 256 threads; rows past the
// descriptor's range read as zero, chunks past D are zeroed.
template <int ROWS, int CW>
struct Tile32 {
  static constexpr int CH = CW / 4;                   // chunks per row
  static constexpr int N = (ROWS * CH + 255) / 256;   // chunks per thread
  static constexpr int RS = rs32(CW);
  int voff[N], loff[N];
  bool zero[N], live[N], swap[N];
  __device__ __forceinline__ void init(int tid, int64_t row_stride, int D) {
#pragma unroll
    for (int it = 0; it < N; ++it) {
      const int ci = it * 256 + tid, r = ci / CH, c4 = ci - r * CH;
      live[it] = ROWS * CH % 256 == 0 || ci < ROWS * CH;
      voff[it] = (int)(r * row_stride * 4) + 16 * c4;
      loff[it] = r * RS + 4 * c4;
      zero[it] = 4 * c4 >= D;
      swap[it] = (r & 8) != 0;
    }
  }
  __device__ __forceinline__ void load(__amdgpu_buffer_rsrc_t rs, int soff, u32x4 (&x)[N]) const {
#pragma unroll
    for (int it = 0; it < N; ++it)
      if (live[it]) x[it] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rs, voff[it], soff, 0));
  }
  __device__ __forceinline__ void store(float* dst, const u32x4 (&x)[N]) const {
#pragma unroll
    for (int it = 0; it < N; ++it) {
      if (!live[it]) continue;
      u32x4 v = zero[it] ? (u32x4){0u, 0u, 0u, 0u} : x[it];
      if (swap[it]) v = (u32x4){v[2], v[3], v[0], v[1]};
      *(u32x4*)(dst + loff[it]) = v;
    }
  }
};

// Four mask elements of one row as exp2-domain addends (keys key4 .. key4+3,
// key4 a multiple of 4, the row's readable span a whole number of 8-key
// runs): one 4-, 8- or 16-byte read.  Bool zeros become -inf.
__device__ __forceinline__ f32x4 mask_run4(__amdgpu_buffer_rsrc_t rs, int row_off, int key4, int kind) {
  f32x4 a;
  if (kind == MASK_BOOL) {
    const uint32_t w = __builtin_amdgcn_raw_buffer_load_b32(rs, row_off + key4, 0, 0);
#pragma unroll
    for (int i = 0; i < 4; ++i) a[i] = ((w >> (8 * i)) & 0xffu) ? 0.f : -INFINITY;
  } else if (kind == MASK_F32) {
    a = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(rs, row_off + 4 * key4, 0, 0)) * kLog2e;
  } else {
    const u32x2 w = __builtin_bit_cast(u32x2, __builtin_amdgcn_raw_buffer_load_b64(rs, row_off + 2 * key4, 0, 0));
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const f32x2 f = kind == MASK_F16 ? Elt<_Float16>::unpack(w[i]) : Elt<__bf16>::unpack(w[i]);
      a[2 * i] = f[0] * kLog2e;
      a[2 * i + 1] = f[1] * kLog2e;
    }
  }
  return a;
}

// ---- Delta_i = sum_d dO_id * O_id, 8 lanes per row (D a multiple of 4)
__global__ void __launch_bounds__(256) attn_bwd32_delta(const BwdParams p) {
  const int sub = thread_x() & 7;
  const int64_t g = (int64_t)block_x() * 32 + (thread_x() >> 3);  // row over B*H*Sq
  const bool live = g < (int64_t)p.B * p.H * p.Sq;
  float acc = 0.f;
  if (live) {
    const int64_t bh = g / p.Sq;
    const int i = (int)(g - bh * p.Sq);
    const int b = (int)(bh / p.H), h = (int)(bh - (int64_t)b * p.H);
    const float* orow = (const float*)p.o + b * p.o_b + h * p.o_h + (int64_t)i * p.o_s;
    const float* drow = (const float*)p.dout + b * p.do_b + h * p.do_h + (int64_t)i * p.do_s;
    for (int c4 = sub; 4 * c4 < p.D; c4 += 8) {
      const f32x4 a = *(const f32x4*)(orow + 4 * c4);
      const f32x4 d = *(const f32x4*)(drow + 4 * c4);
#pragma unroll
      for (int e = 0; e < 4; ++e) acc = __builtin_fmaf(a[e], d[e], acc);
    }
  }
  acc += __shfl_xor(acc, 1, 8);
  acc += __shfl_xor(acc, 2, 8);
  acc += __shfl_xor(acc, 4, 8);
  if (live && sub == 0) p.delta[g] = acc;
}

// Store a [16 rows x NDB*16 columns] set of transposed accumulators (lane
// (l16, g), block db: row `row`, columns 16 db + 4 g .. + 3) times `mul`.
template <int NDB>
__device__ __forceinline__ void store_rows32(float* base, int64_t row_stride, int row, int nrows, int D, int g,
                                             const f32x4 (&acc)[NDB], float mul) {
  if (row >= nrows) return;
  float* dst = base + (int64_t)row * row_stride;
#pragma unroll
  for (int db = 0; db < NDB; ++db) {
    const int d = 16 * db + 4 * g;
    if (d < D) *(f32x4*)(dst + d) = acc[db] * mul;
  }
}

// ---- dK, dV for one block of 64 keys (4 waves x 16 keys), sweeping 32-row
// query tiles (Q, dO, lse, Delta) through double-buffered LDS, one barrier
// per tile.  Grouped-query K/V: the sweep runs over every query head of the
// K/V head's group, so the group's contributions add up in registers.
template <int DK, bool CAUSAL>
__global__ void __launch_bounds__(256) attn_bwd32_dkdv(const BwdParams p) {
  constexpr int BQ = 32, BKV = 64;
  constexpr int NKS = DK / 4;            // k-steps of S and dP
  constexpr int NDB = (DK + 15) / 16;    // 16-column blocks of dK and dV
  constexpr int CW = NDB * 16;           // tile columns (zero past D)
  using Tile = Tile32<BQ, CW>;
  constexpr int RS = Tile::RS;
  __shared__ __attribute__((aligned(16))) float lds[2 * 2 * BQ * RS];  // [slot][Q, dO][row][col]
  // [slot][lse2, Delta][row]: lse2 = lse * log2 e (+inf for rows past Sq or
  // rows that saw no key: P = 0 there)
  __shared__ __attribute__((aligned(16))) float lsd[2][2][BQ];

  const int tid = thread_x(), wave = tid >> 6, lane = tid & 63, l16 = lane & 15, g = lane >> 4;
  // (batch, K/V head) and key block; split sweeps: (block, part) pairs as
  // virtual blocks.  Causal: longest sweeps first (kv_tile)
  const int ns = p.nsplit > 1 ? p.nsplit : 1;
  int bhk, kb, part;
  {
    int bh0, vb;
    kv_tile(block_x(), p.B * p.Hkv, p.n_blk * ns, CAUSAL, bh0, vb);
    bhk = __builtin_amdgcn_readfirstlane(bh0);
    vb = __builtin_amdgcn_readfirstlane(vb);
    kb = __builtin_amdgcn_readfirstlane(vb / ns);
    part = vb - kb * ns;
  }
  const int b = __builtin_amdgcn_readfirstlane(bhk / p.Hkv), hk = bhk - b * p.Hkv;
  const int Sq = p.Sq, Sk = p.Sk, D = p.D;
  const int kw0 = kb * BKV + wave * 16;  // first key of this wave
  const int key = kw0 + l16;             // this lane's key

  // B operands held for the sweep: K (negative scale folded into its sign)
  // and V of this lane's key, one head-dim column per k-step
  const float* kg = (const float*)p.k + b * p.k_b + hk * p.k_h;
  const float* vg = (const float*)p.v + b * p.v_b + hk * p.v_h;
  const float ksign = p.sign ? -1.f : 1.f;
  float kf[NKS], vf[NKS];
#pragma unroll
  for (int s = 0; s < NKS; ++s) {
    const int d = 4 * s + g;
    const bool in = key < Sk && d < D;
    kf[s] = in ? ksign * kg[(int64_t)key * p.k_s + d] : 0.f;
    vf[s] = in ? vg[(int64_t)key * p.v_s + d] : 0.f;
  }

  Tile lq, ldo;
  lq.init(tid, p.q_s, D);
  ldo.init(tid, p.do_s, D);
  const int sb = sbase(l16, g, RS);
  int tb[4];
#pragma unroll
  for (int r = 0; r < 4; ++r) tb[r] = tbase(l16, g, r, RS);

  f32x4 dva[NDB], dka[NDB];
#pragma unroll
  for (int db = 0; db < NDB; ++db) dva[db] = dka[db] = (f32x4){};

  // the sweep: query tiles t0 .. t1-1 of each query head of the group as one
  // sequence of nj tiles, of which this workgroup takes [jb, je) (all of it
  // unless the sweep is split); (fg, ft) = head and tile of the next fetch,
  // (cg, ct) those of the tile being computed
  const int t0 = CAUSAL ? kb * (BKV / BQ) : 0;  // earlier query tiles see none of the block's keys
  const int t1 = (Sq + BQ - 1) / BQ;
  const int nt = t1 > t0 ? t1 - t0 : 0;
  const int nj = nt * p.group;
  const int jb = (int)((int64_t)part * nj / ns), je = (int)((int64_t)(part + 1) * nj / ns);
  const int jg0 = nt > 0 ? jb / nt : 0;
  u32x4 xq[Tile::N], xd[Tile::N];
  float xl = INFINITY, xdl = 0.f;
  const int h0 = hk * p.group;
  int fg = jg0, ft = t0 + (jb - jg0 * nt);
  auto fetch = [&]() {
    const int h = h0 + fg;
    const float* qg = (const float*)p.q + b * p.q_b + h * p.q_h;
    const float* dog = (const float*)p.dout + b * p.do_b + h * p.do_h;
    const __amdgpu_buffer_rsrc_t qrs = uniform_rsrc(qg, ((int64_t)(Sq - 1) * p.q_s + D) * 4);
    const __amdgpu_buffer_rsrc_t dors = uniform_rsrc(dog, ((int64_t)(Sq - 1) * p.do_s + D) * 4);
    const int q0 = ft * BQ;
    lq.load(qrs, (int)(q0 * p.q_s * 4), xq);
    ldo.load(dors, (int)(q0 * p.do_s * 4), xd);
    if (tid < BQ) {
      const int row = q0 + tid;
      const int64_t hoff = ((int64_t)b * p.H + h) * Sq;
      xl = INFINITY;
      xdl = 0.f;
      if (row < Sq) {
        const float L = p.lse[hoff + row];
        xl = L > -INFINITY ? L * kLog2e : INFINITY;
        xdl = p.delta[hoff + row];
      }
    }
    if (++ft == t1) {
      ft = t0;
      ++fg;
    }
  };
  auto put = [&](int slot) {
    float* base = lds + slot * 2 * BQ * RS;
    lq.store(base, xq);
    ldo.store(base + BQ * RS, xd);
    if (tid < BQ) {
      lsd[slot][0][tid] = xl;
      lsd[slot][1][tid] = xdl;
    }
  };

  float* dkg = (float*)p.dk + b * p.dk_b + hk * p.dk_h;
  float* dvg = (float*)p.dv + b * p.dv_b + hk * p.dv_h;
  // the result: gradients, or this part's partial rows (dK unscaled)
  auto finish = [&]() {
    if (ns > 1) {
      const int64_t rows = (int64_t)p.B * p.Hkv * Sk;
      float* const pk = p.part + ((int64_t)part * p.B * p.Hkv + bhk) * Sk * D;
      store_rows32<NDB>(pk, D, key, Sk, D, g, dka, 1.f);
      store_rows32<NDB>(pk + ns * rows * D, D, key, Sk, D, g, dva, 1.f);
    } else {
      store_rows32<NDB>(dvg, p.dv_s, key, Sk, D, g, dva, 1.f);
      store_rows32<NDB>(dkg, p.dk_s, key, Sk, D, g, dka, p.scale);
    }
  };
  if (je == jb) {  // no query of this range sees the block (causal): zeros
    finish();
    return;
  }
  const bool masked = p.mask_kind != MASK_NONE;
  const int mes = masked ? mask_bytes(p.mask_kind) : 1;
  const float c = p.c;
  fetch();
  put(0);
  lds_barrier();
  int cg = jg0, ct = t0 + (jb - jg0 * nt);
  for (int j = jb; j < je; ++j) {
    const int slot = (j - jb) & 1;
    if (j + 1 < je) fetch();
    const int q0 = ct * BQ;
    const float* qs = lds + slot * 2 * BQ * RS;
    const float* dos = qs + BQ * RS;
    __amdgpu_buffer_rsrc_t mrs = uniform_rsrc(p.q, 0);
    if (masked) {
      const int h = h0 + cg;
      mrs = uniform_rsrc((const char*)p.mask + (b * p.m_b + h * p.m_h) * mes,
                         ((int64_t)(Sq - 1) * p.m_q + (Sk + 7) / 8 * 8) * mes);
    }
#pragma unroll
    for (int qb = 0; qb < BQ / 16; ++qb) {
      const int qlo = q0 + 16 * qb;
      // causal: a block whose last query precedes this wave's first key adds nothing
      if (CAUSAL && qlo + 15 < kw0) continue;
      f32x4 s = (f32x4){}, dp = (f32x4){};
#pragma unroll
      for (int st = 0; st < NKS; ++st) {
        const int pos = sb + 16 * qb * RS + 4 * st;
        s = mma4(qs[pos], kf[st], s);
        dp = mma4(dos[pos], vf[st], dp);
      }
      // s: S[query qlo + 4g + i][key]
      const f32x4 l2 = *(const f32x4*)&lsd[slot][0][16 * qb + 4 * g];
      const f32x4 dl = *(const f32x4*)&lsd[slot][1][16 * qb + 4 * g];
      float x[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) x[i] = __builtin_fmaf(s[i], c, -l2[i]);
      if (masked) {
        if (p.m_q == 0 || Sq == 1) {  // one row for every query: one element per lane
          const float a = mask_elem(mrs, key * mes, p.mask_kind);
#pragma unroll
          for (int i = 0; i < 4; ++i) x[i] += a;
        } else {
#pragma unroll
          for (int i = 0; i < 4; ++i)
            x[i] += mask_elem(mrs, (int)(((int64_t)(qlo + 4 * g + i) * p.m_q + key) * mes), p.mask_kind);
        }
      }
      // causal diagonal: one wave-uniform branch around the four checks
      if (CAUSAL && qlo < kw0 + 15) {
#pragma unroll
        for (int i = 0; i < 4; ++i)
          if (key > qlo + 4 * g + i) x[i] = -INFINITY;
      }
      float pp[4], ds[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        pp[i] = fast_exp2(x[i]);
        ds[i] = pp[i] * (dp[i] - dl[i]);
      }
      // dV^T += dO^T P, dK^T += Q^T dS: k-step r takes queries 4g + r
#pragma unroll
      for (int r = 0; r < 4; ++r)
#pragma unroll
        for (int db = 0; db < NDB; ++db) {
          const int pos = tb[r] + 16 * qb * RS + 16 * db;
          dva[db] = mma4(dos[pos], pp[r], dva[db]);
          dka[db] = mma4(qs[pos], ds[r], dka[db]);
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

// ---- dQ for one block of 64 queries (4 waves x 16 queries), sweeping
// 32-key tiles of K and V through double-buffered LDS.
template <int DK, bool CAUSAL>
__global__ void __launch_bounds__(256) attn_bwd32_dq(const BwdParams p) {
  constexpr int BQ = 64, BK = 32;
  constexpr int NKS = DK / 4;
  constexpr int NDB = (DK + 15) / 16;
  constexpr int CW = NDB * 16;
  using Tile = Tile32<BK, CW>;
  constexpr int RS = Tile::RS;
  __shared__ __attribute__((aligned(16))) float lds[2 * 2 * BK * RS];  // [slot][K, V][row][col]

  const int tid = thread_x(), wave = tid >> 6, lane = tid & 63, l16 = lane & 15, g = lane >> 4;
  // split sweeps: (query block, part) pairs as ns virtual blocks per block
  const int ns = p.nsplit_q > 1 ? p.nsplit_q : 1;
  int bh, qblk, part;
  {
    FwdParams fp;
    fp.B = p.B; fp.H = p.H; fp.n_qblk = p.n_blk * ns; fp.n_wg = p.n_wg;
    int vblk;
    wg_tile(block_x(), fp, CAUSAL, bh, vblk);  // causal: longest key sweeps first
    qblk = vblk / ns;
    part = vblk - qblk * ns;
  }
  const int b = bh / p.H, h = bh - b * p.H;
  const int Sq = p.Sq, Sk = p.Sk, D = p.D;
  const int qw0 = qblk * BQ + wave * 16;
  const int qrow = qw0 + l16;  // this lane's query

  // B operands held for the sweep: Q (negative scale folded into its sign)
  // and dO of this lane's query
  const float* qg = (const float*)p.q + b * p.q_b + h * p.q_h;
  const float* dog = (const float*)p.dout + b * p.do_b + h * p.do_h;
  const float qsign = p.sign ? -1.f : 1.f;
  float qf[NKS], dof[NKS];
#pragma unroll
  for (int s = 0; s < NKS; ++s) {
    const int d = 4 * s + g;
    const bool in = qrow < Sq && d < D;
    qf[s] = in ? qsign * qg[(int64_t)qrow * p.q_s + d] : 0.f;
    dof[s] = in ? dog[(int64_t)qrow * p.do_s + d] : 0.f;
  }
  // rows past Sq, and rows that saw no key in the forward: P = 0
  const float L = qrow < Sq ? p.lse[(int64_t)bh * Sq + qrow] : -INFINITY;
  const float l2 = L > -INFINITY ? L * kLog2e : INFINITY;
  const float dl = qrow < Sq ? p.delta[(int64_t)bh * Sq + qrow] : 0.f;
  const bool masked = p.mask_kind != MASK_NONE;
  const int mes = masked ? mask_bytes(p.mask_kind) : 1;
  const __amdgpu_buffer_rsrc_t mrs =
      uniform_rsrc(masked ? (const void*)((const char*)p.mask + (b * p.m_b + h * p.m_h) * mes) : p.q,
                   masked ? ((int64_t)(Sq - 1) * p.m_q + (Sk + 7) / 8 * 8) * mes : 0);
  const int mrow = masked ? (int)((int64_t)min(qrow, Sq - 1) * p.m_q * mes) : 0;

  const int hk = h / p.group;
  const float* kg = (const float*)p.k + b * p.k_b + hk * p.k_h;
  const float* vg = (const float*)p.v + b * p.v_b + hk * p.v_h;
  const __amdgpu_buffer_rsrc_t krs = uniform_rsrc(kg, ((int64_t)(Sk - 1) * p.k_s + D) * 4);
  const __amdgpu_buffer_rsrc_t vrs = uniform_rsrc(vg, ((int64_t)(Sk - 1) * p.v_s + D) * 4);
  Tile lk, lv;
  lk.init(tid, p.k_s, D);
  lv.init(tid, p.v_s, D);
  const int sb = sbase(l16, g, RS);
  int tb[4];
#pragma unroll
  for (int r = 0; r < 4; ++r) tb[r] = tbase(l16, g, r, RS);

  f32x4 dqa[NDB];
#pragma unroll
  for (int db = 0; db < NDB; ++db) dqa[db] = (f32x4){};

  const int kend = CAUSAL ? min(Sk, qblk * BQ + BQ) : Sk;  // keys any row of the block sees
  const int nt = (kend + BK - 1) / BK;
  const int wlast = qw0 + 15;  // this wave's last query
  u32x4 xk[Tile::N], xv[Tile::N];
  auto fetch = [&](int t) {
    lk.load(krs, (int)(t * BK * p.k_s * 4), xk);
    lv.load(vrs, (int)(t * BK * p.v_s * 4), xv);
  };
  auto put = [&](int slot) {
    float* base = lds + slot * 2 * BK * RS;
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
    const float* ks = lds + slot * 2 * BK * RS;
    const float* vs = ks + BK * RS;
#pragma unroll
    for (int kb = 0; kb < BK / 16; ++kb) {
      const int k0 = t * BK + 16 * kb;
      if (CAUSAL && k0 > wlast) continue;  // keys past this wave's last query add nothing
      f32x4 s = (f32x4){}, dp = (f32x4){};
#pragma unroll
      for (int st = 0; st < NKS; ++st) {
        const int pos = sb + 16 * kb * RS + 4 * st;
        s = mma4(ks[pos], qf[st], s);
        dp = mma4(vs[pos], dof[st], dp);
      }
      // s: S^T[key k0 + 4g + i][query]
      float x[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) x[i] = __builtin_fmaf(s[i], c, -l2);
      if (masked) {
        const f32x4 a = mask_run4(mrs, mrow, k0 + 4 * g, p.mask_kind);
#pragma unroll
        for (int i = 0; i < 4; ++i) x[i] += a[i];
      }
      // keys past Sk, and the causal diagonal: one wave-uniform branch
      if (k0 + 16 > Sk || (CAUSAL && k0 + 15 > qw0)) {
        const int lim = CAUSAL ? min(Sk, qrow + 1) : Sk;  // keys below lim count
#pragma unroll
        for (int i = 0; i < 4; ++i)
          if (k0 + 4 * g + i >= lim) x[i] = -INFINITY;
      }
      float ds[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) ds[i] = fast_exp2(x[i]) * (dp[i] - dl);
      // dQ^T += K^T dS^T: k-step r takes keys 4g + r
#pragma unroll
      for (int r = 0; r < 4; ++r)
#pragma unroll
        for (int db = 0; db < NDB; ++db)
          dqa[db] = mma4(ks[tb[r] + 16 * kb * RS + 16 * db], ds[r], dqa[db]);
    }
    if (t + 1 < kt1) put(slot ^ 1);
    lds_barrier();
  }

  if (ns > 1) {  // this part's partial rows, unscaled
    store_rows32<NDB>(p.part_q + ((int64_t)part * p.B * p.H + bh) * Sq * D, D, qrow, Sq, D, g, dqa, 1.f);
    return;
  }
  float* dqg = (float*)p.dq + b * p.dq_b + h * p.dq_h;
  store_rows32<NDB>(dqg, p.dq_s, qrow, Sq, D, g, dqa, p.scale);
}

template <int DK, bool CAUSAL>
hipError_t launch_bwd32_t(const BwdParams& p0, hipStream_t s) {
  BwdParams p = p0;
  const int64_t rows = (int64_t)p.B * p.H * p.Sq;
  hipLaunchKernelGGL(attn_bwd32_delta, dim3((unsigned)((rows + 31) / 32)), dim3(256), 0, s, p);
  p.n_blk = (p.Sk + 63) / 64;
  const int ns = p.nsplit > 1 && p.part ? p.nsplit : 1;
  p.nsplit = ns;
  p.n_wg = p.B * p.Hkv * p.n_blk * ns;
  hipLaunchKernelGGL((attn_bwd32_dkdv<DK, CAUSAL>), dim3(p.n_wg), dim3(256), 0, s, p);
  if (ns > 1) launch_part_sums<float>(p, true, s);
  p.n_blk = (p.Sq + 63) / 64;
  const int nsq = p.nsplit_q > 1 && p.part_q ? p.nsplit_q : 1;
  p.nsplit_q = nsq;
  p.n_wg = p.B * p.H * p.n_blk * nsq;
  hipLaunchKernelGGL((attn_bwd32_dq<DK, CAUSAL>), dim3(p.n_wg), dim3(256), 0, s, p);
  if (nsq > 1) launch_part_sums<float>(p, false, s);
  return hipGetLastError();
}

template <bool CAUSAL>
hipError_t launch_bwd32_dk(const BwdParams& p, int dk, hipStream_t s) {
  switch (dk) {
    case 32: return launch_bwd32_t<32, CAUSAL>(p, s);
    case 40: return launch_bwd32_t<40, CAUSAL>(p, s);
    case 64: return launch_bwd32_t<64, CAUSAL>(p, s);
    case 96: return launch_bwd32_t<96, CAUSAL>(p, s);
    case 128: return launch_bwd32_t<128, CAUSAL>(p, s);
    case 192: return launch_bwd32_t<192, CAUSAL>(p, s);
    case 256: return launch_bwd32_t<256, CAUSAL>(p, s);
  }
  return hipErrorNotSupported;
}

}  // namespace

int bwd32_bucket(int D) {
  for (int dk : {32, 40, 64, 96, 128, 192, 256})
    if (D <= dk) return dk;
  return -1;
}

// Split plan of the fp32 gradient sweeps (split_sweep): dK/dV over 64-key
// blocks sweeping 32-query tiles, dQ over 64-query blocks sweeping 32-key
// tiles.  Workgroups per CU from the kernels' registers and LDS: dK/dV 5 at
// D <= 32, 4 up to 40, 3 (causal 4) up to 64, 2 up to 128, then 1; dQ 7, 5,
// 4, 3 up to 96, 2 up to 128, then 1.
BwdSplit bwd32_split(int B, int H, int Hkv, int Sq, int Sk, int D, bool causal, int cus) {
  BwdSplit sp;
  const int dk = bwd32_bucket(D);
  if (dk < 0 || (int64_t)B * H * Sq == 0 || Hkv < 1) return sp;
  const int occ_kv = dk <= 32 ? 5 : dk <= 40 ? 4 : dk <= 64 ? (causal ? 4 : 3) : dk <= 128 ? 2 : 1;
  const int occ_q = dk <= 32 ? 7 : dk <= 40 ? 5 : dk <= 64 ? 4 : dk <= 96 ? 3 : dk <= 128 ? 2 : 1;
  sp.ns_kv = split_sweep((int64_t)B * Hkv * ((Sk + 63) / 64), occ_kv, cus, causal,
                         (int64_t)(H / Hkv) * ((Sq + 31) / 32));
  sp.ns_q = split_sweep((int64_t)B * H * ((Sq + 63) / 64), occ_q, cus, causal, (Sk + 31) / 32);
  return sp;
}

hipError_t launch_bwd32(const BwdParams& p, bool causal, hipStream_t s) {
  if ((int64_t)p.B * p.H * p.Sq == 0) return hipSuccess;
  const int dk = bwd32_bucket(p.D);
  return causal ? launch_bwd32_dk<true>(p, dk, s) : launch_bwd32_dk<false>(p, dk, s);
}

}  // namespace cmpext3
