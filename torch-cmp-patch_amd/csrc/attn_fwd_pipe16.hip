// Instantiations and tile table of the software-pipelined fp16/bf16 kernel
// (template in attn_fwd_pipe16.h), used for head dims up to 128.
//
// Like the v2 table in attn_fwd_mfma16.hip this replaces the reference's
// per-head-dim template table (src/cuda/fp16_flash_attention_hfma2.cu:278-285);
// entries come from an offline sweep on an MI355X.  All buckets use 4-wave
// workgroups and 32-key tiles; the waves per SIMD are the most the registers
// allow without spilling (D = 32: 4, D <= 64: 3, D <= 128: 2).
#include <stdio.h>

#include "attn_fwd_pipe16.h"

namespace cmpext3 {

namespace {

constexpr int kPipeNw = 4;
constexpr int kPipeBk = 32;
constexpr int pipe_occ(int dk) { return dk <= 32 ? 4 : dk <= 64 ? 3 : 2; }

template <typename T, int DK, bool CAUSAL, bool PRESCALE>
hipError_t launch_dk(const FwdParams& p, hipStream_t s) {
  // OPT 1: s_setprio around the MFMA block; OPT 8: zero K columns past D
  if (p.D == DK) return launch_pipe16_cfg<T, DK, kPipeNw, kPipeBk, pipe_occ(DK), CAUSAL, PRESCALE, 1>(p, s);
  return launch_pipe16_cfg<T, DK, kPipeNw, kPipeBk, pipe_occ(DK), CAUSAL, PRESCALE, 1 | 8>(p, s);
}

template <typename T, bool CAUSAL, bool PRESCALE>
hipError_t launch_bucket(const FwdParams& p, int dk, hipStream_t s) {
  switch (dk) {
    case 32: return launch_dk<T, 32, CAUSAL, PRESCALE>(p, s);
    case 48: return launch_dk<T, 48, CAUSAL, PRESCALE>(p, s);
    case 64: return launch_dk<T, 64, CAUSAL, PRESCALE>(p, s);
    case 80: return launch_dk<T, 80, CAUSAL, PRESCALE>(p, s);
    case 96: return launch_dk<T, 96, CAUSAL, PRESCALE>(p, s);
    case 128: return launch_dk<T, 128, CAUSAL, PRESCALE>(p, s);
  }
  return hipErrorNotSupported;
}

}  // namespace

// True when the pipelined kernel takes this problem: head-dim bucket <= 128,
// a key sweep long enough for its prologue (four tiles in flight) to pay off
// (SDXL cross-attention, Sk = 77, is faster on the v2 kernel), and K/V tiles
// addressable with 32-bit buffer offsets.
constexpr int kPipeMinSk = 256;

bool pipe16_applies(const FwdParams& p, int dk) {
  if (dk > 128 || p.Sk < kPipeMinSk) return false;
  const int64_t rs = p.k_s > p.v_s ? p.k_s : p.v_s;
  return (int64_t)(p.Sk + kPipeBk) * rs * 2 < (int64_t(1) << 31);
}

// `prescale` applies to fp16 (Q * scale * log2(e) must stay finite).  bf16
// never pre-scales: rounding Q*c to 8 mantissa bits moves each score by up to
// 2^-9 of its size, which at scale 1 (scores of tens of log2 units) breaks
// the 2e-2 bf16 bar, so bf16 scores get one FMA each instead.
hipError_t launch_pipe16(const FwdParams& p, int dk, bool bf16, bool causal, bool prescale, hipStream_t s) {
  if (bf16)
    return causal ? launch_bucket<__bf16, true, false>(p, dk, s) : launch_bucket<__bf16, false, false>(p, dk, s);
  if (prescale)
    return causal ? launch_bucket<_Float16, true, true>(p, dk, s) : launch_bucket<_Float16, false, true>(p, dk, s);
  return causal ? launch_bucket<_Float16, true, false>(p, dk, s) : launch_bucket<_Float16, false, false>(p, dk, s);
}

void describe_pipe16(int dk, int Sq, char* buf, int len) {
  const int bq = kPipeNw * 32;
  snprintf(buf, len,
           "pipe16 mfma 32x32x16 S^T-form, K one tile ahead of V: DK=%d DP=%d waves=%d BQ=%d BK=%d "
           "waves/SIMD=%d qtiles=%d",
           dk, (dk + 31) / 32 * 32, kPipeNw, bq, kPipeBk, pipe_occ(dk), (Sq + bq - 1) / bq);
}

}  // namespace cmpext3
