// Instantiations, tile table and key-split plan of the software-pipelined
// fp16/bf16 kernel (template in attn_fwd_pipe16.h), used for head dims up to
// 128, and for the unmasked inference prefills above 128 (instantiations in
// attn_fwd_pipe16w.hip).
//
// Like the v2 table in attn_fwd_mfma16.hip this replaces the reference's
// per-head-dim template table (src/cuda/fp16_flash_attention_hfma2.cu:278-285);
// entries come from an offline sweep on an MI355X.  All buckets use 4-wave
// workgroups and 32-key tiles; the waves per SIMD are the most the registers
// allow without spilling (D = 32: 4, D <= 64: 3, D <= 128: 2; above 128 one,
// with accumulation registers as the spill space).
//
// The key split (no counterpart in the reference) needs exchange space, and
// the library allocates none: the workspace entry points take it from the
// caller (cmpext3_attn_fwd_workspace_size says how much), the
// allocation-free entry point uses a fixed per-device array in this file
// (`scratch` below), and every other call runs unsplit.  bind_exchange, the
// one place a plan meets its space, serves all the split kernels.
#include <stdio.h>

#include <mutex>

#include "attn_fwd_pipe16.h"

namespace cmpext3 {

namespace {

constexpr int kPipeNw = 4;
constexpr int kPipeBk = 32;
constexpr int pipe_occ(int dk) { return dk <= 32 ? 4 : dk <= 64 ? 3 : dk <= 128 ? 2 : 1; }
// masked launches need a few more registers: D = 32 drops to 3 waves per SIMD
constexpr int pipe_occ_masked(int dk) { return dk <= 64 ? 3 : 2; }

// Split plan limits: a part scans at least kMinPartTiles key tiles (shorter
// parts spend more on their prologue and merge than they save); with no
// whole round a CU holds at most kMaxPartsPerCu parts at once.
constexpr int kMinPartTiles = 8;
constexpr int kMaxPartsPerCu = 2;
constexpr int kMaxCausalParts = 8;       // parts per causal block at most
constexpr int kMinCausalPartTiles = 16;  // tiles of a causal block's longest part at least
constexpr int kLongCausalTiles = 64;     // a long causal sweep (the last block's tiles)
constexpr int kMi355xCus = 256;  // used when no device is visible (host-only calls)

int n_blocks(int B, int H, int Sq) { return B * H * ((Sq + kPipeNw * 32 - 1) / (kPipeNw * 32)); }
int n_key_tiles(int Sk) { return (Sk + kPipeBk - 1) / kPipeBk; }
// Key tiles of query block `nb - 1`'s sweep: all of them, or under causal
// those up to the block's last query row.
int causal_tiles(int Sk, int nb, bool causal) {
  const int64_t kend = causal ? (int64_t)nb * kPipeNw * 32 : Sk;
  return n_key_tiles(kend < Sk ? (int)kend : Sk);
}

// ---- Exchange storage of the allocation-free entry point
//
// One fixed array per device in the library's code object, zero-filled when
// the code object is loaded on a device and never allocated or freed by the
// library: the counters, then 16 MiB of partial (O, m, l) vectors (the
// layout of every exchange space, attn_common.h).  Every allocation-free
// call on a device shares it.  Host code never passes `scratch` itself to a
// kernel (in host code the name is only a stand-in for the device symbol):
// the device address comes from hipGetSymbolAddress, once per device.
constexpr size_t kScratchWsBytes = size_t(16) << 20;
constexpr size_t kScratchBytes = kExchangeCounterBytes + kScratchWsBytes;
static __device__ __align__(256) unsigned char scratch[kScratchBytes];

// This device's scratch address, looked up on the first call with the device
// current (a failed lookup is retried on the next call; until one succeeds
// the allocation-free calls run unsplit).  Nothing is launched: the code
// object's zero fill is the counters' initial state.
void* scratch_ptr() {
  static std::mutex mu;
  static void* ptrs[64] = {};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) {
    (void)hipGetLastError();
    return nullptr;
  }
  std::lock_guard<std::mutex> lock(mu);
  if (!ptrs[dev]) {
    void* ptr = nullptr;
    if (hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)) != hipSuccess) {
      (void)hipGetLastError();
      return nullptr;
    }
    ptrs[dev] = ptr;
  }
  return ptrs[dev];
}

// Waves per block that hold query rows: all of them unless the launch is a
// single block shorter than the workgroup (decode, packed grouped-query rows).
int exchange_waves(int n_qblk, int Sq) {
  return n_qblk > 1 ? kPipeNw : (Sq + 31) / 32 < kPipeNw ? (Sq + 31) / 32 : kPipeNw;
}

// Which blocks run whole and how the rest are cut.  n blocks on `cus` CUs at
// `occ` workgroups per CU; the dispatcher hands workgroup i to CU i mod cus
// while all of them fit, so after the whole rounds each CU takes exactly one
// part.  ntiles: key tiles of a block (causal: of the longest block, whose
// sweep reaches the last query; ntiles_min those of the shortest, the first
// query block's).
//
// Causal launches keep their longest-first order.  Where the blocks fill at
// most half of the workgroup slots and either leave more than half of the
// CUs without a block or sweep long key ranges (at least kLongCausalTiles
// tiles for the last block), every block is cut into the same number of
// parts so that one round holds them all, the longest part keeping at least
// kMinCausalPartTiles tiles: each block's longest part, and so the launch,
// gets shorter.  Measured on MI355X (same run): [1,4,8192,128] bf16 135 ->
// 98 us, [1,8,2048,256] 85 -> 73 us, [1,16,2048,64] fp16 30 -> 25 us,
// [1,8,1024,64] 17 -> 14 us; shorter sweeps on busy CUs lost to the parts'
// prologues and merges ([1,32,1024,128] 25 -> 28 us, [1,32,512,128] 16 ->
// 18 us) and stay whole.  Every part of every block keeps at least one tile
// (a causal row sees a key in the first tile of a part, or none of the part's
// keys: its state then has no weight in the merge).
SplitArgs split_plan(int n, int ntiles, int occ, int cus, bool causal, int ntiles_min) {
  SplitArgs sa = {n, 1, nullptr, nullptr, kPipeNw};
  if (cus <= 0) return sa;
  if (causal) {
    const int slots = occ * cus;
    if (n * 2 > slots || (n * 2 > cus && ntiles < kLongCausalTiles)) return sa;
    int parts = slots / n;
    if (parts > ntiles / kMinCausalPartTiles) parts = ntiles / kMinCausalPartTiles;
    if (parts > ntiles_min) parts = ntiles_min;
    if (parts > kMaxCausalParts) parts = kMaxCausalParts;
    if (parts < 2) return sa;
    sa.nfull = 0;
    sa.nparts = parts;
    return sa;
  }
  const int full = n / cus, rem = n - full * cus;
  if (rem == 0 || full + 1 > occ) return sa;  // whole rounds, or more than fits at once
  // After whole rounds each CU takes one part of the round that remains.  With
  // no whole round (fewer blocks than CUs: decode, short sweeps) each CU can
  // hold several parts at once: more key ranges streamed side by side, more
  // loads in flight (a decode step with one part per CU reaches ~5.2 TB/s).
  const int per_cu = full == 0 ? (occ < kMaxPartsPerCu ? occ : kMaxPartsPerCu) : 1;
  int parts = per_cu * cus / rem;
  if (parts > ntiles / kMinPartTiles) parts = ntiles / kMinPartTiles;
  if (parts < 2) return sa;
  sa.nfull = full * cus;
  sa.nparts = parts;
  return sa;
}

// Stream-K (OPT 512): for non-causal, unmasked inference launches of the
// LDS-DMA buckets whose blocks fill at least the CUs but not whole rounds of
// the occ * cus workgroup slots.  The launch is then ceil(n / slots) rounds
// of workgroups, each taking an equal share of the n * ntiles block-tile
// sequence (with the classic plan the CUs of the last round would idle once
// their half-blocks end: SDXL self-attention, 640 blocks on 768 slots).
// Shares of fewer than kMinPartTiles tiles would spend more on prologues and
// merges than they balance; the counters take 2 per (block, wave).
constexpr int kMaxStreamkWaves = kExchangeCounters / 2;

bool streamk_applies(const FwdParams& p, int n, int dk, int occ, int cus, bool causal) {
  if (causal || p.lse || p.elem_rows || p.mask_kind != MASK_NONE || p.pack_sq > 0) return false;
  if (!(dk == 32 || dk == 64 || dk == 128) || p.Sq <= (kPipeNw - 2) * 32) return false;
  const int slots = occ * cus;
  if (cus <= 0 || n < cus || n % slots == 0 || n * kPipeNw > kMaxStreamkWaves) return false;
  // Only where the classic plan leaves slots idle for the whole launch: one
  // partial round of whole CUs (n a multiple of the CU count: no block left
  // to split), or, at two workgroups per CU, a last round at most half full.
  // Where the classic plan splits the blocks past the whole CUs, it measured
  // faster (SDXL self-attention 91.1 us against 97.7 us stream-K, same run:
  // every stream-K share pays a second prologue and every block a merge);
  // [2,4,4096,4096,64], one block per CU, 54.6 us unsplit against 44.8 us.
  const bool idle_round = n < slots && n % cus == 0;
  const bool thin_tail = n > slots && occ == 2 && n % slots <= slots / 2;
  if (!idle_round && !thin_tail) return false;
  const int64_t rounds = (n + slots - 1) / slots;
  return (int64_t)n * n_key_tiles(p.Sk) / (rounds * slots) >= kMinPartTiles;
}

// The stream-K launch: workgroup count and part slots per block (an upper
// bound on the shares one block's tiles can touch).
SplitArgs streamk_plan(int n, int ntiles, int occ, int cus) {
  const int slots = occ * cus;
  const int W = (n + slots - 1) / slots * slots;
  const int share = (int)((int64_t)n * ntiles / W);  // tiles per share, rounded down
  SplitArgs sa = {0, ntiles / share + 2, nullptr, nullptr, kPipeNw, W};
  return sa;
}

// The mask is the same for every query row and is read in whole runs.
bool mask_bcast(const FwdParams& p) {
  return p.mask_kind != MASK_NONE && !p.mask_narrow && (p.m_q == 0 || p.Sq == 1);
}

template <typename T, int DK, bool CAUSAL, bool PRESCALE, int MOPT>
hipError_t launch_dk(const FwdParams& p, const SplitArgs& sa, hipStream_t s) {
  // OPT 1: s_setprio around the MFMA blocks; OPT 8: zero K columns past D;
  // OPT 16 (MOPT): attention mask
  constexpr int occ = MOPT ? pipe_occ_masked(DK) : pipe_occ(DK);
  // OPT 128: a single query block whose last waves hold no rows (decode,
  // packed query groups); those waves become the only K/V loaders and the
  // waves with rows only compute.  Taken with at least two rowless waves (the
  // loaders' chunk split assumes 128 or more loader threads); decode steps
  // run 0-20% faster than with every wave loading and computing.
  if constexpr (!CAUSAL && MOPT == 0) {
    if (p.Sq <= (kPipeNw - 2) * 32) {
      if (p.D == DK) return launch_pipe16_cfg<T, DK, kPipeNw, kPipeBk, occ, CAUSAL, PRESCALE, 1 | 128>(p, sa, s);
      return launch_pipe16_cfg<T, DK, kPipeNw, kPipeBk, occ, CAUSAL, PRESCALE, 1 | 8 | 128>(p, sa, s);
    }
  }
  // OPT 256 | 2: unmasked launches of the 32 / 64 / 128 buckets load K/V
  // tiles straight into swizzled LDS (no staging registers, one load
  // instruction per 2 KiB of tile, no bank conflicts; 3-4% faster on SDXL
  // self-attention, 6% on causal bf16 D = 128 than register staging).
  if constexpr (MOPT == 0 && (DK == 32 || DK == 64 || DK == 128)) {
    // OPT 512: stream-K (equal shares of the block-tile sequence; see
    // attn_fwd_pipe16.h), planned by launch_pipe16
    if constexpr (!CAUSAL) {
      if (sa.sk_wgs > 0) {
        if (p.D == DK) return launch_pipe16_cfg<T, DK, kPipeNw, kPipeBk, occ, CAUSAL, PRESCALE, 1 | 2 | 256 | 512>(p, sa, s);
        return launch_pipe16_cfg<T, DK, kPipeNw, kPipeBk, occ, CAUSAL, PRESCALE, 1 | 2 | 8 | 256 | 512>(p, sa, s);
      }
    }
    if (p.D == DK) return launch_pipe16_cfg<T, DK, kPipeNw, kPipeBk, occ, CAUSAL, PRESCALE, 1 | 2 | 256>(p, sa, s);
    return launch_pipe16_cfg<T, DK, kPipeNw, kPipeBk, occ, CAUSAL, PRESCALE, 1 | 2 | 8 | 256>(p, sa, s);
  }
  // masked launches of those buckets: the same LDS DMA, whose freed staging
  // registers the mask words use (masked fp16 D = 64 spilled 3-21 registers
  // with register staging; SDXL self-attention with a key-padding mask
  // 162 -> 121 us with the mask test of attn_fwd_pipe16.h)
  if constexpr (MOPT != 0 && (DK == 32 || DK == 64 || DK == 128)) {
    // OPT 1024: a query-broadcast mask read in runs (key padding [B,1,1,Sk]
    // and the like): its tile slices ride the DMA ring, no loads in the step
    if (mask_bcast(p)) {
      if (p.D == DK) return launch_pipe16_cfg<T, DK, kPipeNw, kPipeBk, occ, CAUSAL, PRESCALE, 1 | 2 | 256 | 1024 | MOPT>(p, sa, s);
      return launch_pipe16_cfg<T, DK, kPipeNw, kPipeBk, occ, CAUSAL, PRESCALE, 1 | 2 | 8 | 256 | 1024 | MOPT>(p, sa, s);
    }
    if (p.D == DK) return launch_pipe16_cfg<T, DK, kPipeNw, kPipeBk, occ, CAUSAL, PRESCALE, 1 | 2 | 256 | MOPT>(p, sa, s);
    return launch_pipe16_cfg<T, DK, kPipeNw, kPipeBk, occ, CAUSAL, PRESCALE, 1 | 2 | 8 | 256 | MOPT>(p, sa, s);
  }
  if (p.D == DK) return launch_pipe16_cfg<T, DK, kPipeNw, kPipeBk, occ, CAUSAL, PRESCALE, 1 | MOPT>(p, sa, s);
  return launch_pipe16_cfg<T, DK, kPipeNw, kPipeBk, occ, CAUSAL, PRESCALE, 1 | 8 | MOPT>(p, sa, s);
}

// Training forward (OPT 32: write the row log-sum-exp; MOPT 16: with an
// attention mask): buckets 64 and 128 only.
template <typename T, bool CAUSAL, bool PRESCALE, int MOPT>
hipError_t launch_lse_m(const FwdParams& p, const SplitArgs& sa, int dk, hipStream_t s) {
  // K/V straight into swizzled LDS, as for inference; query-broadcast masks
  // with K (OPT 1024)
  constexpr int LD = 2 | 256;
  if constexpr (MOPT != 0) {
    if (mask_bcast(p)) {
      if (dk == 64) {
        if (p.D == 64)
          return launch_pipe16_cfg<T, 64, kPipeNw, kPipeBk, pipe_occ(64), CAUSAL, PRESCALE, 1 | 32 | MOPT | LD | 1024>(p, sa, s);
        return launch_pipe16_cfg<T, 64, kPipeNw, kPipeBk, pipe_occ(64), CAUSAL, PRESCALE, 1 | 8 | 32 | MOPT | LD | 1024>(p, sa, s);
      }
      if (dk == 128) {
        if (p.D == 128)
          return launch_pipe16_cfg<T, 128, kPipeNw, kPipeBk, pipe_occ(128), CAUSAL, PRESCALE, 1 | 32 | MOPT | LD | 1024>(p, sa, s);
        return launch_pipe16_cfg<T, 128, kPipeNw, kPipeBk, pipe_occ(128), CAUSAL, PRESCALE, 1 | 8 | 32 | MOPT | LD | 1024>(p, sa, s);
      }
      return hipErrorNotSupported;
    }
  }
  if (dk == 64) {
    if (p.D == 64)
      return launch_pipe16_cfg<T, 64, kPipeNw, kPipeBk, pipe_occ(64), CAUSAL, PRESCALE, 1 | 32 | MOPT | LD>(p, sa, s);
    return launch_pipe16_cfg<T, 64, kPipeNw, kPipeBk, pipe_occ(64), CAUSAL, PRESCALE, 1 | 8 | 32 | MOPT | LD>(p, sa, s);
  }
  if (dk == 128) {
    if (p.D == 128)
      return launch_pipe16_cfg<T, 128, kPipeNw, kPipeBk, pipe_occ(128), CAUSAL, PRESCALE, 1 | 32 | MOPT | LD>(p, sa, s);
    return launch_pipe16_cfg<T, 128, kPipeNw, kPipeBk, pipe_occ(128), CAUSAL, PRESCALE, 1 | 8 | 32 | MOPT | LD>(p, sa, s);
  }
  return hipErrorNotSupported;
}

template <typename T, bool CAUSAL, bool PRESCALE>
hipError_t launch_lse(const FwdParams& p, const SplitArgs& sa, int dk, hipStream_t s) {
  return p.mask_kind != MASK_NONE ? launch_lse_m<T, CAUSAL, PRESCALE, 16>(p, sa, dk, s)
                                  : launch_lse_m<T, CAUSAL, PRESCALE, 0>(p, sa, dk, s);
}

// Narrow rows (OPT 64, FwdParams::elem_rows 4 or 8): inference, masked
// (MOPT 16) or not, buckets 64 and 128 only (other head dims are zero-padded
// up to them).
template <typename T, bool CAUSAL, int MOPT = 0>
hipError_t launch_narrow(const FwdParams& p, const SplitArgs& sa, int dk, hipStream_t s) {
  constexpr int occ64 = MOPT ? pipe_occ_masked(64) : pipe_occ(64);
  constexpr int occ128 = MOPT ? pipe_occ_masked(128) : pipe_occ(128);
  if (dk == 64)
    return launch_pipe16_cfg<T, 64, kPipeNw, kPipeBk, occ64, CAUSAL, false, 1 | 64 | MOPT>(p, sa, s);
  if (dk == 128)
    return launch_pipe16_cfg<T, 128, kPipeNw, kPipeBk, occ128, CAUSAL, false, 1 | 64 | MOPT>(p, sa, s);
  return hipErrorNotSupported;
}

template <typename T, bool CAUSAL, bool PRESCALE, int MOPT = 0>
hipError_t launch_bucket(const FwdParams& p, const SplitArgs& sa, int dk, hipStream_t s) {
  switch (dk) {
    case 32: return launch_dk<T, 32, CAUSAL, PRESCALE, MOPT>(p, sa, s);
    case 48: return launch_dk<T, 48, CAUSAL, PRESCALE, MOPT>(p, sa, s);
    case 64: return launch_dk<T, 64, CAUSAL, PRESCALE, MOPT>(p, sa, s);
    case 80: return launch_dk<T, 80, CAUSAL, PRESCALE, MOPT>(p, sa, s);
    case 96: return launch_dk<T, 96, CAUSAL, PRESCALE, MOPT>(p, sa, s);
    case 128: return launch_dk<T, 128, CAUSAL, PRESCALE, MOPT>(p, sa, s);
  }
  return hipErrorNotSupported;
}


}  // namespace

hipError_t launch_pipe16_wide(const FwdParams& p, const SplitArgs& sa, int dk, bool bf16, bool causal,
                              bool prescale, hipStream_t s);

// Compute units of the current device (256 on MI355X), cached per device.
int device_cus() {
  static int cus[64] = {};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) {
    (void)hipGetLastError();
    return kMi355xCus;
  }
  if (cus[dev] == 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) {
      (void)hipGetLastError();
      return kMi355xCus;
    }
    cus[dev] = n;
  }
  return cus[dev];
}

int bind_exchange(const FwdParams& p, int parts, size_t part_bytes, int ncnt, f32x4** ws, int** cnt) {
  *ws = nullptr;
  *cnt = nullptr;
  if (parts < 2) return 1;
  // the space this call may use: the fixed scratch, or the caller's workspace
  void* base = nullptr;
  size_t bytes = 0;
  if (p.dry) {
    p.dry->need = kExchangeCounterBytes + (size_t)parts * part_bytes;
    bytes = p.fixed_exchange ? kScratchBytes : p.workspace_bytes;
  } else if (p.fixed_exchange) {
    base = scratch_ptr();
    bytes = base ? kScratchBytes : 0;
  } else if (p.workspace) {
    base = p.workspace;
    bytes = p.workspace_bytes;
  }
  // as many key ranges as the partials room holds, if the counters fit
  int fit = 0;
  if (bytes > kExchangeCounterBytes && ncnt <= kExchangeCounters && part_bytes > 0) {
    const size_t room = (bytes - kExchangeCounterBytes) / part_bytes;
    fit = room < (size_t)parts ? (int)room : parts;
  }
  if (fit < 2) fit = 1;
  if (p.dry) {
    p.dry->parts = fit;
    return fit;
  }
  if (fit >= 2) {
    *cnt = (int*)base;
    *ws = (f32x4*)((char*)base + kExchangeCounterBytes);
  }
  return fit;
}

// True when the pipelined kernel takes this problem: head-dim bucket <= 128,
// a key sweep long enough for its prologue (four tiles in flight) to pay off
// (shorter sweeps run faster on the short-key and v2 kernels) unless an
// attention mask or the log-sum-exp output is asked for (up to D = 128 only
// this kernel has them), and K/V tiles addressable with 32-bit buffer
// offsets.  Above D = 128: launches with whole-chunk rows whose query
// blocks hold rows in at least three of their four waves (fewer rows: the
// decode and packed-row paths) and sweep at least kPipeMinSk keys, masked or
// not, inference or training.
constexpr int kPipeMinSk = 256;

bool pipe16_applies(const FwdParams& p, int dk) {
  if (dk > 128 && (p.elem_rows || p.Sq <= (kPipeNw - 2) * 32 || p.Sk < kPipeMinSk)) return false;
  if (p.Sk < kPipeMinSk && p.mask_kind == MASK_NONE && !p.lse) return false;
  const int64_t rs = p.k_s > p.v_s ? p.k_s : p.v_s;
  return (int64_t)(p.Sk + kPipeBk) * rs * 2 < (int64_t(1) << 31);
}

// `prescale` applies to fp16 (Q * scale * log2(e) must stay finite).  bf16
// never pre-scales: rounding Q*c to 8 mantissa bits moves each score by up to
// 2^-9 of its size, which at scale 1 (scores of tens of log2 units) breaks
// the 2e-2 bf16 bar, so bf16 scores get one FMA each instead.
// Grouped-query launches whose query heads hold less than one block of rows
// each (decode, short prefills) pack the G query heads of a K/V head into the
// rows of one problem: the K/V of that head is then streamed once for all of
// them, instead of once per query head with mostly empty blocks.  Non-causal,
// unmasked, inference launches only (the row position then does not matter).
constexpr int kPackMaxSq = 64;

bool packs_query_heads(const FwdParams& p, bool causal) {
  return !causal && p.kv_group > 1 && p.Sq <= kPackMaxSq && p.mask_kind == MASK_NONE && !p.lse &&
         p.pack_sq == 0 && (int64_t)p.kv_group * p.Sq <= (int64_t)INT32_MAX / 2;
}

void pack_query_heads(FwdParams& p) {
  const int G = p.kv_group;
  p.pack_sq = p.Sq;
  p.q_g = p.q_h;
  p.o_g = p.o_h;
  p.q_h *= G;  // packed head hk starts at query head hk * G
  p.o_h *= G;
  p.H /= G;
  p.Sq *= G;
  p.kv_group = 1;
}

hipError_t launch_pipe16(const FwdParams& p0, int dk0, bool bf16, bool causal, bool prescale, hipStream_t s) {
  FwdParams p = p0;
  if (packs_query_heads(p, causal)) pack_query_heads(p);
  // the training forward and the narrow-row variants have the 64 and 128
  // buckets only up to D = 128; above it the training forward has 192 and
  // 256, and neither it nor masked launches pre-scale Q (one instantiation
  // per dtype)
  const int dk = dk0 > 128 ? (p.lse && dk0 < 192 ? 192 : dk0)
                           : (p.lse || p.elem_rows) ? (dk0 <= 64 ? 64 : 128) : dk0;
  if (dk > 128 && (p.lse || p.mask_kind != MASK_NONE)) prescale = false;
  if (p.elem_rows && (p.elem_rows < 4 || p.lse)) return hipErrorNotSupported;
  // Without pre-scaling, masked keys enter as raw -inf and meet the multiplier
  // c in one FMA; scale 0 would make that 0 * -inf.  A multiplier of 1e-30
  // instead leaves every finite score's exp2 argument within 1e-22 of -m,
  // which rounds to the same probability as scale 0 gives, and keeps -inf.
  if ((!prescale || p.elem_rows) && p.c == 0.f) p.c = 1e-30f;
  const int cus = device_cus();
  const int occ = p.mask_kind != MASK_NONE ? pipe_occ_masked(dk) : pipe_occ(dk);
  const int n = n_blocks(p.B, p.H, p.Sq);
  const int dp = (dk + 31) / 32 * 32;
  // stream-K where it applies and its exchange fits the space this call has
  size_t sk_need = 0;
  if (streamk_applies(p, n, dk, occ, cus, causal)) {
    SplitArgs sk = streamk_plan(n, n_key_tiles(p.Sk), occ, cus);
    const size_t part_bytes = (size_t)n * kPipeNw * split_vectors(dp) * 64 * sizeof(f32x4);
    const int fit = bind_exchange(p, sk.nparts, part_bytes, 2 * n * kPipeNw, &sk.ws, &sk.cnt);
    if (p.dry) sk_need = p.dry->need;
    if (fit == sk.nparts) {
      if (p.dry) return hipSuccess;
      return bf16 ? launch_bucket<__bf16, false, false>(p, sk, dk, s)
                  : prescale ? launch_bucket<_Float16, false, true>(p, sk, dk, s)
                             : launch_bucket<_Float16, false, false>(p, sk, dk, s);
    }
  }
  const int n_qblk = (p.Sq + kPipeNw * 32 - 1) / (kPipeNw * 32);
  SplitArgs sa = split_plan(n, causal_tiles(p.Sk, n_qblk, causal), occ, cus, causal, causal_tiles(p.Sk, 1, causal));
  sa.nwl = exchange_waves((p.Sq + kPipeNw * 32 - 1) / (kPipeNw * 32), p.Sq);
  if (p.dry) *p.dry = SplitInfo{0, 1};  // the stream-K attempt's record, if any, is not this plan
  if (sa.nparts > 1) {
    // Exchange space: the fixed scratch or the caller's workspace, cut to
    // fewer key ranges when the plan does not fit it (an unsplit launch needs
    // none, so no problem is ever refused for want of space).  The plan keeps
    // its whole blocks; only the split blocks' part count changes.
    const int nsplit = n - sa.nfull;
    const size_t part_bytes = (size_t)nsplit * sa.nwl * split_vectors(dp) * 64 * sizeof(f32x4);
    sa.nparts = bind_exchange(p, sa.nparts, part_bytes, 2 * nsplit * sa.nwl, &sa.ws, &sa.cnt);
    if (sa.nparts < 2) sa = SplitArgs{n, 1, nullptr, nullptr, sa.nwl};
  }
  if (p.dry) {
    // the size query reports the best plan's need (stream-K's, when it applies)
    if (sk_need > p.dry->need) p.dry->need = sk_need;
    return hipSuccess;
  }
  if (dk > 128) return launch_pipe16_wide(p, sa, dk, bf16, causal, prescale, s);
  if (p.lse) {  // training forward, masked or not
    if (bf16) return causal ? launch_lse<__bf16, true, false>(p, sa, dk, s) : launch_lse<__bf16, false, false>(p, sa, dk, s);
    if (prescale)
      return causal ? launch_lse<_Float16, true, true>(p, sa, dk, s) : launch_lse<_Float16, false, true>(p, sa, dk, s);
    return causal ? launch_lse<_Float16, true, false>(p, sa, dk, s) : launch_lse<_Float16, false, false>(p, sa, dk, s);
  }
  if (p.elem_rows) {  // never pre-scaled: the narrow fp16 kernels then spill
    if (p.mask_kind != MASK_NONE) {
      if (bf16)
        return causal ? launch_narrow<__bf16, true, 16>(p, sa, dk, s) : launch_narrow<__bf16, false, 16>(p, sa, dk, s);
      return causal ? launch_narrow<_Float16, true, 16>(p, sa, dk, s)
                    : launch_narrow<_Float16, false, 16>(p, sa, dk, s);
    }
    if (bf16)
      return causal ? launch_narrow<__bf16, true>(p, sa, dk, s) : launch_narrow<__bf16, false>(p, sa, dk, s);
    return causal ? launch_narrow<_Float16, true>(p, sa, dk, s) : launch_narrow<_Float16, false>(p, sa, dk, s);
  }
  if (p.mask_kind != MASK_NONE) {  // with causal, a pair must pass both rules
    if (bf16)
      return causal ? launch_bucket<__bf16, true, false, 16>(p, sa, dk, s)
                    : launch_bucket<__bf16, false, false, 16>(p, sa, dk, s);
    if (prescale)
      return causal ? launch_bucket<_Float16, true, true, 16>(p, sa, dk, s)
                    : launch_bucket<_Float16, false, true, 16>(p, sa, dk, s);
    return causal ? launch_bucket<_Float16, true, false, 16>(p, sa, dk, s)
                  : launch_bucket<_Float16, false, false, 16>(p, sa, dk, s);
  }
  if (bf16)
    return causal ? launch_bucket<__bf16, true, false>(p, sa, dk, s) : launch_bucket<__bf16, false, false>(p, sa, dk, s);
  if (prescale)
    return causal ? launch_bucket<_Float16, true, true>(p, sa, dk, s) : launch_bucket<_Float16, false, true>(p, sa, dk, s);
  return causal ? launch_bucket<_Float16, true, false>(p, sa, dk, s) : launch_bucket<_Float16, false, false>(p, sa, dk, s);
}

void describe_pipe16(int dk, int B, int H, int Sq, int Sk, bool causal, bool narrow, char* buf, int len) {
  const int bq = kPipeNw * 32;
  const int n = n_blocks(B, H, Sq);
  const int n_qblk = (Sq + bq - 1) / bq;
  const SplitArgs sa = split_plan(n, causal_tiles(Sk, n_qblk, causal), pipe_occ(dk), device_cus(), causal,
                                  causal_tiles(Sk, 1, causal));
  char split[96] = "";
  FwdParams p = {};
  p.Sq = Sq;
  p.Sk = Sk;
  p.mask_kind = MASK_NONE;
  p.elem_rows = narrow ? 4 : 0;
  if (streamk_applies(p, n, dk, pipe_occ(dk), device_cus(), causal)) {
    const SplitArgs sk = streamk_plan(n, n_key_tiles(Sk), pipe_occ(dk), device_cus());
    snprintf(split, sizeof split, " stream-K: %d workgroups x %lld tiles of %d blocks (with a workspace)", sk.sk_wgs,
             (long long)n * n_key_tiles(Sk) / sk.sk_wgs, n);
  } else if (sa.nparts > 1) {
    snprintf(split, sizeof split, " key-split: %d whole + %d x %d parts", sa.nfull, n - sa.nfull, sa.nparts);
  }
  snprintf(buf, len,
           "pipe16 mfma 32x32x16 S^T-form, K one tile ahead of V: DK=%d DP=%d waves=%d BQ=%d BK=%d "
           "waves/SIMD=%d qtiles=%d%s",
           dk, (dk + 31) / 32 * 32, kPipeNw, bq, kPipeBk, pipe_occ(dk), (Sq + bq - 1) / bq, split);
}

}  // namespace cmpext3
