// Instantiations and tile table of the fp16/bf16 MFMA attention kernel
// (kernel template in attn_fwd_mfma16.h), and the fp16/bf16 entry point:
// head dims up to 128, and unmasked inference prefills above 128, go to the
// software-pipelined kernel (attn_fwd_pipe16.hip); the other launches above
// 128 (masked, training, few query rows, short key sweeps), and K/V row
// strides too large for its 32-bit buffer offsets, run this one.
//
// The tile table replaces the reference's hard-coded per-head-dim template
// table (src/cuda/fp16_flash_attention_hfma2.cu:278-285) and its build-time
// autotune idea (setup.py:54-123): entries were chosen by an offline sweep on
// an MI355X; nothing is measured at build or run time.
#include <stdio.h>
#include <string.h>

#include "attn_fwd_mfma16.h"

namespace cmpext3 {

namespace {

struct Tile16 {
  int nw, qb, bk, occ;  // waves/WG, 32-row query blocks per wave, keys per tile, waves/SIMD
};

// Head-dim buckets; D is zero-padded up to the bucket inside the kernel.
const int kMfma16Dk[] = {32, 48, 64, 80, 96, 128, 160, 192, 256};

// Measured on MI355X (SDXL fp16 D=64 and Qwen3 bf16 D=128 shapes): three
// 4-wave workgroups per CU beat two for D <= 96; at D = 128 two workgroups
// with 64-key tiles win; larger head dims need the registers of one.
constexpr Tile16 tile16(int dk) {
  return dk <= 96 ? Tile16{4, 1, 64, 3} : dk <= 128 ? Tile16{4, 1, 64, 2} : Tile16{4, 1, 32, 1};
}

// OPT 1: s_setprio(1) around the MFMA blocks (padded LDS rows, max-first
// rescale); OPT 16: attention mask; OPT 64: element-granular rows
// (FwdParams::elem_rows)
template <typename T, int DK, bool CAUSAL, bool PRESCALE, int EOPT>
hipError_t launch_dk(const FwdParams& p, hipStream_t s) {
  constexpr Tile16 tt = tile16(DK);
  return launch_mfma16_cfg<T, DK, tt.nw, tt.qb, tt.bk, tt.occ, CAUSAL, PRESCALE, 1 | EOPT>(p, s);
}

template <typename T, bool CAUSAL, bool PRESCALE, int EOPT = 0>
hipError_t launch_bucket(const FwdParams& p, int dk, hipStream_t s) {
  switch (dk) {
    case 32: return launch_dk<T, 32, CAUSAL, PRESCALE, EOPT>(p, s);
    case 48: return launch_dk<T, 48, CAUSAL, PRESCALE, EOPT>(p, s);
    case 64: return launch_dk<T, 64, CAUSAL, PRESCALE, EOPT>(p, s);
    case 80: return launch_dk<T, 80, CAUSAL, PRESCALE, EOPT>(p, s);
    case 96: return launch_dk<T, 96, CAUSAL, PRESCALE, EOPT>(p, s);
    case 128: return launch_dk<T, 128, CAUSAL, PRESCALE, EOPT>(p, s);
    case 160: return launch_dk<T, 160, CAUSAL, PRESCALE, EOPT>(p, s);
    case 192: return launch_dk<T, 192, CAUSAL, PRESCALE, EOPT>(p, s);
    case 256: return launch_dk<T, 256, CAUSAL, PRESCALE, EOPT>(p, s);
  }
  return hipErrorInvalidValue;
}

// attention-masked launches (OPT bit 16) of the head dims above 128; EOPT 64:
// narrow rows
template <typename T, bool CAUSAL, bool PRESCALE, int EOPT = 0>
hipError_t launch_masked(const FwdParams& p, int dk, hipStream_t s) {
  switch (dk) {
    case 160: return launch_dk<T, 160, CAUSAL, PRESCALE, 16 | EOPT>(p, s);
    case 192: return launch_dk<T, 192, CAUSAL, PRESCALE, 16 | EOPT>(p, s);
    case 256: return launch_dk<T, 256, CAUSAL, PRESCALE, 16 | EOPT>(p, s);
  }
  return hipErrorInvalidValue;
}

// training forwards (OPT bit 32: the row log-sum-exp) of the head dims above
// 128, masked (OPT bit 16) or not, in the backward's buckets 192 and 256; no
// pre-scaled Q, so one instantiation per dtype serves every scale
template <typename T, bool CAUSAL>
hipError_t launch_train(const FwdParams& p, int dk, hipStream_t s) {
  const bool m = p.mask_kind != MASK_NONE;
  if (dk <= 192)
    return m ? launch_dk<T, 192, CAUSAL, false, 32 | 16>(p, s) : launch_dk<T, 192, CAUSAL, false, 32>(p, s);
  return m ? launch_dk<T, 256, CAUSAL, false, 32 | 16>(p, s) : launch_dk<T, 256, CAUSAL, false, 32>(p, s);
}

}  // namespace

bool pipe16_applies(const FwdParams& p, int dk);
bool short16_applies(const FwdParams& p, int dk, bool causal);
hipError_t launch_short16(const FwdParams& p, int dk, bool bf16, hipStream_t s);
void describe_short16(int dk, int Sq, int Sk, char* buf, int len);
hipError_t launch_pipe16(const FwdParams& p, int dk, bool bf16, bool causal, bool prescale, hipStream_t s);
void describe_pipe16(int dk, int B, int H, int Sq, int Sk, bool causal, bool narrow, char* buf, int len);
bool packs_query_heads(const FwdParams& p, bool causal);
void pack_query_heads(FwdParams& p);
bool decode16_applies(const FwdParams& p, bool causal);
hipError_t launch_decode16(const FwdParams& p, bool bf16, hipStream_t s);
void describe_decode16(int D, int B, int H, int Sq, int Sk, char* buf, int len);

int mfma16_bucket(int D) {
  for (int dk : kMfma16Dk)
    if (D <= dk) return dk;
  return -1;
}

// Q can be pre-scaled by scale*log2(e) without overflow when |c| <= 1; that
// path is taken for fp16 (for bf16 the scaled Q would keep only 8 mantissa bits).
static bool use_prescale(const FwdParams& p, bool bf16) { return !bf16 && p.c <= 1.0f; }

// Head-dim > 128 prefills go to the pipelined kernel except causal launches
// of the 192 bucket without pre-scaled Q: there this kernel's instantiation
// fits two waves per SIMD (252 registers) and measured faster on MI355X
// (bf16 [1,32/8,4096,4096,192] causal 221 against 254 us, same run; fp16
// pre-scaled, at one wave per SIMD here, 307 against 266 us).
static bool keeps_wide(int dk, bool causal, bool prescale) { return dk == 192 && causal && !prescale; }

hipError_t launch_mfma16(const FwdParams& p0, bool bf16, bool causal, hipStream_t s) {
  const int dk = mfma16_bucket(p0.D);
  if (dk < 0) return hipErrorInvalidValue;
  // decode steps (few query rows per K/V head) above the pipelined kernel's
  // head dims, and below them where the key split must cut deep: every wave
  // streams its own key tiles (attn_fwd_decode16.hip)
  if (decode16_applies(p0, causal)) return launch_decode16(p0, bf16, s);
  // grouped-query launches with few query rows that stay on this kernel run
  // over K/V heads with the group's query rows packed into one problem (the
  // pipelined kernel packs for itself)
  FwdParams p = p0;
  const bool pack = packs_query_heads(p0, causal) && !short16_applies(p0, dk, causal) &&
                    !((!p0.elem_rows || p0.elem_rows >= 4) && pipe16_applies(p0, dk));
  if (pack) pack_query_heads(p);
  if (p.elem_rows) {
    // narrow rows (inference; the ABI sends training calls here only with
    // whole aligned chunks, and masked ones only in 4- or 8-byte pieces): 4-
    // or 8-byte pieces on the pipelined kernel where it applies, else this
    // kernel in any piece size (masked: head dims above 128)
    if (p.lse) return hipErrorNotSupported;
    if (p.elem_rows >= 4 && pipe16_applies(p, dk))
      return launch_pipe16(p, dk, bf16, causal, use_prescale(p, bf16), s);
    if (p.mask_kind != MASK_NONE) {
      if (dk <= 128) return hipErrorNotSupported;
      return bf16 ? (causal ? launch_masked<__bf16, true, false, 64>(p, dk, s)
                            : launch_masked<__bf16, false, false, 64>(p, dk, s))
                  : (causal ? launch_masked<_Float16, true, false, 64>(p, dk, s)
                            : launch_masked<_Float16, false, false, 64>(p, dk, s));
    }
    if (bf16)
      return causal ? launch_bucket<__bf16, true, false, 64>(p, dk, s)
                    : launch_bucket<__bf16, false, false, 64>(p, dk, s);
    return causal ? launch_bucket<_Float16, true, false, 64>(p, dk, s)
                  : launch_bucket<_Float16, false, false, 64>(p, dk, s);
  }
  if (short16_applies(p, dk, causal)) return launch_short16(p, dk, bf16, s);
  if (pipe16_applies(p, dk) && !keeps_wide(dk, causal, use_prescale(p, bf16)))
    return launch_pipe16(p, dk, bf16, causal, use_prescale(p, bf16), s);
  // training forwards reach this kernel above D = 128 only (the pipelined
  // kernel writes the log-sum-exp up to 128); masked launches likewise
  if (p.lse) {
    if (dk <= 128) return hipErrorNotSupported;
    if (bf16) return causal ? launch_train<__bf16, true>(p, dk, s) : launch_train<__bf16, false>(p, dk, s);
    return causal ? launch_train<_Float16, true>(p, dk, s) : launch_train<_Float16, false>(p, dk, s);
  }
  if (p.mask_kind != MASK_NONE) {
    if (dk <= 128) return hipErrorNotSupported;
    if (bf16)
      return causal ? launch_masked<__bf16, true, false>(p, dk, s) : launch_masked<__bf16, false, false>(p, dk, s);
    if (use_prescale(p, bf16))
      return causal ? launch_masked<_Float16, true, true>(p, dk, s) : launch_masked<_Float16, false, true>(p, dk, s);
    return causal ? launch_masked<_Float16, true, false>(p, dk, s) : launch_masked<_Float16, false, false>(p, dk, s);
  }
  if (bf16)
    return causal ? launch_bucket<__bf16, true, false>(p, dk, s)
                  : launch_bucket<__bf16, false, false>(p, dk, s);
  if (use_prescale(p, bf16))
    return causal ? launch_bucket<_Float16, true, true>(p, dk, s)
                  : launch_bucket<_Float16, false, true>(p, dk, s);
  return causal ? launch_bucket<_Float16, true, false>(p, dk, s)
                : launch_bucket<_Float16, false, false>(p, dk, s);
}

int mfma16_max_bk() { return 64; }

void describe_mfma16(int D, int B, int H, int Sq, int Sk, bool causal, bool bf16, char* buf, int len) {
  const int dk = mfma16_bucket(D);
  FwdParams p = {};
  p.Sk = Sk;
  p.k_s = p.v_s = D;
  p.mask_kind = MASK_NONE;
  // contiguous rows of a D that is not whole 16-byte chunks are narrow: in
  // 4- or 8-byte pieces (D even) on the pipelined kernel where it applies
  const bool elem = D % 8 != 0;
  p.B = B;
  p.H = H;
  p.D = D;
  p.Sq = Sq;
  p.kv_group = 1;
  if (!elem && decode16_applies(p, causal)) {
    describe_decode16(D, B, H, Sq, Sk, buf, len);
    return;
  }
  if (!elem && short16_applies(p, dk, causal)) {
    describe_short16(dk, Sq, Sk, buf, len);
    return;
  }
  // (narrow rows above 128 stay here; the default scale: fp16 pre-scales Q)
  const bool wide = dk > 128;
  if ((!elem || (D % 2 == 0 && !wide)) && pipe16_applies(p, dk) && !(wide && keeps_wide(dk, causal, !bf16))) {
    describe_pipe16(elem ? (dk <= 64 ? 64 : 128) : dk, B, H, Sq, Sk, causal, elem, buf, len);
    if (elem) snprintf(buf + strlen(buf), len - strlen(buf), " narrow rows");
    return;
  }
  const Tile16 t = tile16(dk);
  const int bq = t.nw * t.qb * 32;
  const int n = B * H * ((Sq + bq - 1) / bq);
  const int nwl = Sq > bq ? t.nw : (Sq + 31) / 32 < t.nw ? (Sq + 31) / 32 : t.nw;
  const int64_t nb = (Sq + bq - 1) / bq;
  const int kmax = causal && nb * bq < Sk ? (int)(nb * bq) : Sk, kmin = causal && bq < Sk ? bq : Sk;
  const int parts = split_parts16(n, (kmax + t.bk - 1) / t.bk, t.occ, device_cus(), causal, (dk + 31) / 32 * 32,
                                  nwl < t.nw, (kmin + t.bk - 1) / t.bk);
  char split[48] = "";
  if (parts >= 2) snprintf(split, sizeof split, " key-split: %d x %d parts", n, parts);
  snprintf(buf, len,
           "mfma16 32x32x16 S^T-form: DK=%d DP=%d waves=%d qblocks/wave=%d BQ=%d BK=%d "
           "waves/SIMD=%d qtiles=%d%s%s",
           dk, (dk + 31) / 32 * 32, t.nw, t.qb, bq, t.bk, t.occ, (Sq + bq - 1) / bq, split,
           elem ? " narrow rows" : "");
}

}  // namespace cmpext3
