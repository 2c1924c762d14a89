// Instantiations of the short-key fp16/bf16 kernel (template in
// attn_fwd_short16.h): non-causal, unmasked launches with Sk <= 128 and a
// head-dim bucket <= 128, the SDXL cross-attention shape (Sk = 77) among them.
// Three key capacities (64, 96 and 128 keys) keep the score registers and
// LDS near what the problem needs.
#include <stdio.h>

#include "attn_fwd_short16.h"

namespace cmpext3 {

namespace {

template <typename T, int DK, int NKH>
hipError_t launch_dk(const FwdParams& p, hipStream_t s) {
  // OPT 8: zero K columns past D.  (s_setprio around the MFMAs, OPT 1, measured
  // 4% slower on SDXL cross-attention: each wave runs one short MFMA burst.)
  if (p.D == DK) return launch_short16_cfg<T, DK, NKH>(p, s);
  return launch_short16_cfg<T, DK, NKH, 8>(p, s);
}

template <typename T, int NKH>
hipError_t launch_bucket(const FwdParams& p, int dk, hipStream_t s) {
  switch (dk) {
    case 32: return launch_dk<T, 32, NKH>(p, s);
    case 48: return launch_dk<T, 48, NKH>(p, s);
    case 64: return launch_dk<T, 64, NKH>(p, s);
    case 80: return launch_dk<T, 80, NKH>(p, s);
    case 96: return launch_dk<T, 96, NKH>(p, s);
    case 128: return launch_dk<T, 128, NKH>(p, s);
  }
  return hipErrorNotSupported;
}

// 16-key slices a launch provides for: at least 3 (48 keys), at most 8
int key_slices(int Sk) { return Sk <= 48 ? 3 : (Sk + 15) / 16; }

}  // namespace

bool short16_applies(const FwdParams& p, int dk, bool causal) {
  if (causal || p.mask_kind != MASK_NONE || p.lse || dk > 128 || p.Sk > 128) return false;
  // 32-bit buffer offsets: K/V rows up to the key capacity, Q/O rows up to
  // the last query block's end
  const int64_t rs = p.k_s > p.v_s ? p.k_s : p.v_s;
  const int64_t qs = p.q_s > p.o_s ? p.q_s : p.o_s;
  return (int64_t)128 * rs * 2 < (int64_t(1) << 31) && ((int64_t)p.Sq + 128) * qs * 2 < (int64_t(1) << 31);
}

hipError_t launch_short16(const FwdParams& p, int dk, bool bf16, hipStream_t s) {
  switch (key_slices(p.Sk)) {
    case 3: return bf16 ? launch_bucket<__bf16, 3>(p, dk, s) : launch_bucket<_Float16, 3>(p, dk, s);
    case 4: return bf16 ? launch_bucket<__bf16, 4>(p, dk, s) : launch_bucket<_Float16, 4>(p, dk, s);
    case 5: return bf16 ? launch_bucket<__bf16, 5>(p, dk, s) : launch_bucket<_Float16, 5>(p, dk, s);
    case 6: return bf16 ? launch_bucket<__bf16, 6>(p, dk, s) : launch_bucket<_Float16, 6>(p, dk, s);
    case 7: return bf16 ? launch_bucket<__bf16, 7>(p, dk, s) : launch_bucket<_Float16, 7>(p, dk, s);
  }
  return bf16 ? launch_bucket<__bf16, 8>(p, dk, s) : launch_bucket<_Float16, 8>(p, dk, s);
}

void describe_short16(int dk, int Sq, int Sk, char* buf, int len) {
  snprintf(buf, len,
           "short16 mfma 32x32x16 S^T-form, all keys in LDS, exact row max: DK=%d DP=%d waves=4 BQ=128 "
           "keys<=%d qtiles=%d",
           dk, (dk + 31) / 32 * 32, 16 * key_slices(Sk), (Sq + 127) / 128);
}

}  // namespace cmpext3
