// Shared definitions of the gfx950 attention-forward kernels.
//
// Both kernel families compute O = softmax(scale * Q K^T [+ causal]) V for one
// (batch, head, query-block) per workgroup, streaming K/V tiles through LDS with
// an online (running max / running sum) softmax in the exp2 domain.  The math
// is the one of the reference's flash kernel (Q pre-scaled by scale*log2(e),
// exp2 online softmax, fp32 running max/sum/output, one final 1/l:
// src/cuda/fp16_flash_attention_hfma2.cu:98-109,162-192,216-238), laid out for
// CDNA4 MFMA instead of HFMA2 dot pairs.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace cmpext3 {

struct SplitInfo;

struct FwdParams {
  const void* q;
  const void* k;
  const void* v;
  void* o;
  // element strides of dims {batch, head, seq}; head-dim stride is 1
  int64_t q_b, q_h, q_s;
  int64_t k_b, k_h, k_s;
  int64_t v_b, v_h, v_s;
  int64_t o_b, o_h, o_s;
  int B, H, Sq, Sk, D;
  int kv_group;     // query heads per K/V head (grouped-query attention; 1 = none)
  int n_qblk;       // query blocks per (batch, head)
  int n_wg;         // workgroups launched = B * H * n_qblk
  float c;          // |scale| * log2(e): scores enter exp2 as s * c - m
  uint32_t q_sign;  // sign mask XORed into Q words when scale < 0
  // optional attention mask (torch SDPA attn_mask), element strides for
  // {batch, head, query}; unit stride along keys; kind: MASK_* below
  const void* mask;
  int64_t m_b, m_h, m_q;
  int mask_kind;
  // the mask is read element by element, nothing past key Sk - 1 of a row
  // (any layout with unit key stride); otherwise in runs of 8 keys, every
  // row readable up to Sk rounded up to 8 (16-byte aligned base, strides a
  // multiple of 4 elements, Sk a multiple of 8)
  int mask_narrow;
  // optional [B*H, Sq] fp32 output: natural-log log-sum-exp of each query
  // row's scale * Q K^T over its visible keys (what a backward pass needs to
  // rebuild P); null = not written.  Written by the pipelined kernel only.
  float* lse;
  // grouped-query row packing (pipelined kernel, non-causal): when pack_sq > 0
  // the launch runs over K/V heads, and row r of head hk is query position
  // r % pack_sq of query head hk * G + r / pack_sq; q_h / o_h then step over a
  // whole group of query heads and q_g / o_g over one query head
  int pack_sq;
  int64_t q_g, o_g;
  // host side only: where a key split exchanges its partial results.
  // fixed_exchange != 0: the library's fixed per-device scratch (the
  // allocation-free entry point); otherwise the caller's workspace
  // (workspace_bytes of it; null / too small: fewer key ranges, or none).
  int fixed_exchange;
  void* workspace;
  size_t workspace_bytes;
  // host side only: a dry run (workspace size query, plan description).
  // When set, the launchers record the plan they would launch here and
  // launch nothing.
  SplitInfo* dry;
  // 0 when every row is whole 16-byte chunks at 16-byte aligned addresses;
  // otherwise the piece size in bytes (2, 4 or 8) of the narrow variants
  // (ld_cols16 / ld_cols32): the largest that divides every base pointer,
  // row stride and D * element size
  int elem_rows;
};

// Work-item and workgroup index through the AMDGPU builtins.  Kernel files
// built with -mno-amdgpu-ieee cannot inline the device library's helpers
// behind threadIdx / blockIdx (their IEEE-mode attribute differs): those
// become real calls whose results land in VGPRs, so every tile index after
// them is computed with vector (often quarter-rate) integer instructions.
__device__ __forceinline__ int thread_x() { return (int)__builtin_amdgcn_workitem_id_x(); }
__device__ __forceinline__ int block_x() { return (int)__builtin_amdgcn_workgroup_id_x(); }

// Compute units of the current device (host side; 256 on MI355X).
int device_cus();

// attention-mask element kinds (FwdParams::mask_kind)
constexpr int MASK_NONE = -1;
constexpr int MASK_F16 = 0;   // additive, fp16
constexpr int MASK_BF16 = 1;  // additive, bf16
constexpr int MASK_F32 = 2;   // additive, fp32
constexpr int MASK_BOOL = 3;  // one byte per element, non-zero keeps the pair

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

constexpr float kLog2e = 1.4426950408889634f;
constexpr int kNumXcd = 8;  // MI355X: 8 XCDs, each with its own L2

// The command processor hands workgroup i to XCD i % 8.  Give every XCD one
// contiguous range of logical tiles so that the query blocks of one head, which
// all stream the same K/V, share that XCD's L2.
__device__ __forceinline__ int xcd_remap(int wg, int n) {
  const int x = wg % kNumXcd;
  const int j = wg / kNumXcd;
  const int base = n / kNumXcd;
  const int rem = n % kNumXcd;
  return x * base + (x < rem ? x : rem) + j;
}

// Which (batch*head, query block) workgroup `wg` computes.  Non-causal: the
// xcd_remap ranges, so the query blocks of one head share an XCD's L2.
// Causal: query block j scans j+1 key blocks, so the start order matters.
// When the heads split evenly over the XCDs, XCD x owns heads x, x+8, ... and
// starts their query blocks longest first across those heads; an XCD starts
// its workgroups in order as slots free up, so this is longest-first list
// scheduling per XCD.  Otherwise the whole grid runs longest first, head
// after head within a length, so that every XCD gets its share of long and
// short blocks (each head's blocks then land on 8 / gcd(B*H, 8) XCDs; the
// contiguous per-XCD ranges gave, e.g. for 4 heads, the first XCD the longest
// half of a head and the second its shortest half).
__device__ __forceinline__ void wg_tile(int wg, const FwdParams& p, bool causal, int& bh, int& qblk) {
  const int BH = p.B * p.H;
  if (causal) {
    int r;
    if (BH % kNumXcd == 0) {
      const int x = wg % kNumXcd, i = wg / kNumXcd, hx = BH / kNumXcd;
      r = i / hx;  // query blocks handed out so far on this XCD, per head
      bh = x + kNumXcd * (i - r * hx);
    } else {
      r = wg / BH;
      bh = wg - r * BH;
    }
    qblk = p.n_qblk - 1 - r;
    return;
  }
  const int tile = xcd_remap(wg, p.n_wg);
  bh = tile / p.n_qblk;
  qblk = tile - bh * p.n_qblk;
}

// Which (batch*K/V head, key block) a dK/dV workgroup of the backward computes,
// nvb blocks per head (with split sweeps, (block, part) pairs as virtual
// blocks).  Causal: key block j is seen by every query from j on, so the
// first blocks have the longest sweeps; like wg_tile, when the heads split
// evenly over the XCDs each XCD starts its heads' blocks longest first across
// those heads (list scheduling per XCD), otherwise the whole grid runs
// longest first.  Non-causal: the xcd_remap ranges.
__device__ __forceinline__ void kv_tile(int wg, int BH, int nvb, bool causal, int& bh, int& vb) {
  if (causal) {
    if (BH % kNumXcd == 0) {
      const int x = wg % kNumXcd, i = wg / kNumXcd, hx = BH / kNumXcd;
      vb = i / hx;  // blocks handed out so far on this XCD, per head
      bh = x + kNumXcd * (i - vb * hx);
    } else {
      vb = wg / BH;
      bh = wg - vb * BH;
    }
    return;
  }
  const int tile = xcd_remap(wg, BH * nvb);
  bh = tile / nvb;
  vb = tile - bh * nvb;
}

// max / sum of a value with its partner 32 lanes away (v_permlane32_swap):
// lane L receives {x[L mod 32], x[32 + L mod 32]} in the two results.
__device__ __forceinline__ float xhalf_max(float x) {
  auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float xhalf_sum(float x) {
  auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// Workgroup barrier for LDS traffic only: waits for this wave's LDS operations
// (lgkmcnt) and meets the other waves, but leaves global loads in flight
// (__syncthreads' fences would drain them).  The memory clobber keeps the
// compiler from moving LDS accesses across it.
__device__ __forceinline__ void lds_barrier() {
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

// Wait until at most N vector-memory operations of this wave are in flight
// (they complete in issue order).  Needed for loads that write LDS directly,
// which the compiler does not order against later LDS reads.
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

// Raw buffer descriptor words (gfx9: base, stride 0, num_records, 32-bit raw
// reads), wave-uniform, for loads issued through inline assembly.
__device__ __forceinline__ u32x4 uniform_rsrc_words(const void* base, int64_t bytes) {
  const uint64_t a = (uint64_t)base;
  const uint32_t lo = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)a);
  const uint32_t hi = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)(a >> 32)) & 0xffffu;
  const uint32_t n = (uint32_t)__builtin_amdgcn_readfirstlane((int)bytes);
  return (u32x4){lo, hi, n, 0x00020000u};
}

// 16 bytes per lane from the buffer (voffset + soffset) straight into LDS:
// lane i writes [lds_byte + 16 i, lds_byte + 16 i + 16); an offset outside
// the buffer writes zeros; lanes off in EXEC write nothing.  Issued as inline
// assembly so that the compiler neither waits for these loads before its own
// LDS reads (it cannot tell the ring slots apart) nor counts them: the caller
// orders them with wait_vmcnt and a barrier.  M0 carries the LDS address
// (the compiler writes it; one wait state before the load reads it).
__device__ __forceinline__ void lds_dma16(const u32x4& rs, uint32_t lds_byte, int voff, int soff) {
  asm volatile("s_nop 0\n\tbuffer_load_dwordx4 %0, %1, %2 offen lds"
               ::"v"(voff), "s"(rs), "s"(soff), "{m0}"(lds_byte)
               : "memory");
}

// 4 bytes per lane from the buffer straight into LDS at lds_byte + 4 i (as
// lds_dma16; used for the small per-tile slices of attention masks).
__device__ __forceinline__ void lds_dma4(const u32x4& rs, uint32_t lds_byte, int voff, int soff) {
  asm volatile("s_nop 0\n\tbuffer_load_dword %0, %1, %2 offen lds"
               ::"v"(voff), "s"(rs), "s"(soff), "{m0}"(lds_byte)
               : "memory");
}

// Narrow row access (FwdParams::elem_rows = a, the largest of 2, 4, 8 bytes
// that divides every base pointer, every row stride and the row length D *
// element size): for head dims that are not a whole number of 16-byte chunks
// and for rows or base pointers that are not 16-byte aligned.  A 16-byte
// chunk is assembled from a-byte pieces, each naturally aligned; since the
// row length is a multiple of a, a piece lies wholly inside or wholly past
// the head dim, and pieces past it (n = elements of the chunk inside the
// head dim) are neither read nor written.  No row is read past its head
// dim and nothing is copied.
__device__ __forceinline__ u32x4 ld_cols16(const uint16_t* p, int n, int a) {
  u32x4 x = {0u, 0u, 0u, 0u};
  if (a == 8) {
    const u32x2* q = (const u32x2*)p;
    const u32x2 lo = q[0];  // n >= 4: the chunk's first piece is in the head dim
    x[0] = lo[0];
    x[1] = lo[1];
    if (n > 4) {
      const u32x2 hi = q[1];
      x[2] = hi[0];
      x[3] = hi[1];
    }
  } else if (a == 4) {
    const uint32_t* q = (const uint32_t*)p;
#pragma unroll
    for (int w = 0; w < 4; ++w)
      if (2 * w < n) x[w] = q[w];
  } else {
#pragma unroll
    for (int e = 0; e < 8; ++e)
      if (e < n) x[e >> 1] |= (uint32_t)p[e] << (16 * (e & 1));
  }
  return x;
}
// the first n (<= 4) of 4 packed 16-bit values w to p, in a-byte pieces
__device__ __forceinline__ void st_cols16x4(uint16_t* p, u32x2 w, int n, int a) {
  if (a == 8) {
    *(u32x2*)p = w;  // n == 4
  } else if (a == 4) {
    uint32_t* q = (uint32_t*)p;
    q[0] = w[0];
    if (n > 2) q[1] = w[1];
  } else {
#pragma unroll
    for (int e = 0; e < 4; ++e)
      if (e < n) p[e] = (uint16_t)(w[e >> 1] >> (16 * (e & 1)));
  }
}
__device__ __forceinline__ u32x4 ld_cols32(const float* p, int n) {
  u32x4 x = {0u, 0u, 0u, 0u};
#pragma unroll
  for (int e = 0; e < 4; ++e)
    if (e < n) x[e] = __float_as_uint(p[e]);
  return x;
}

// Key split of the last query blocks: workgroups [0, nfull) take whole
// blocks; the next (n_blocks - nfull) * nparts take one key range each of the
// remaining blocks.  Per (split block, wave) the parts leave their partial
// O, offset and row sum in ws; one part merges them all and puts the two
// counters of the (block, wave) in cnt back to zero (the protocols are in
// attn_fwd_pipe16.h).  nparts == 1: no split, ws/cnt unused.
struct SplitArgs {
  int nfull, nparts;
  f32x4* ws;  // split blocks * nparts * nwl * (float4 vectors per lane) * 64 float4
  int* cnt;   // 2 * split blocks * nwl counters, zero between launches
  // waves per block that hold query rows (and so exchange): NW, or fewer
  // when a single query block is shorter than the workgroup (decode)
  int nwl;
  // stream-K launches of the pipelined kernel: the workgroup count (every
  // block is a possible split block, nparts the part slots per block);
  // 0 otherwise
  int sk_wgs;
};

// float4 vectors each lane of the fp16/bf16 kernels leaves per part: its O
// fragments, then (m, l)
constexpr int split_vectors(int dp) { return dp / 8 + 1; }

// Layout of every exchange space (the caller's workspace and the library's
// fixed scratch alike): kExchangeCounters 32-bit counters first, then the
// partial results.  The counters must be zero before a space's first use;
// every split launch puts the ones it used back to zero, so a space reused
// in stream order, for any problem shape, stays ready.
constexpr int kExchangeCounters = 16384;  // CMPEXT3_WORKSPACE_COUNTER_BYTES / 4
constexpr size_t kExchangeCounterBytes = kExchangeCounters * sizeof(int);

// What a launch would do (FwdParams::dry): the workspace bytes that let its
// full key-split plan run (0: it never splits) and the key ranges per split
// block it takes with the workspace it was given (1: unsplit).
struct SplitInfo {
  size_t need;
  int parts;
};

// Bind a key-split plan to exchange space (host side, attn_fwd_pipe16.hip).
// The plan cuts each of its split blocks into `parts` key ranges; one range
// of all of them takes part_bytes of partials and the plan uses ncnt
// counters.  Returns the key ranges that fit the space FwdParams names (the
// fixed scratch, or the caller's workspace), at most `parts` and 1 when no
// split fits (then the launch runs unsplit), and sets ws / cnt.  A dry run
// records the full plan's need and the part count in p.dry and binds
// nothing.
int bind_exchange(const FwdParams& p, int parts, size_t part_bytes, int ncnt, f32x4** ws, int** cnt);

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

}  // namespace cmpext3
