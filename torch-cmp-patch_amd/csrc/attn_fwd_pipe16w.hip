// Instantiations of the software-pipelined fp16/bf16 kernel (template in
// attn_fwd_pipe16.h) for head dims above 128: unmasked inference prefills of
// the 160, 192 and 256 buckets (plan and dispatch in attn_fwd_pipe16.hip;
// masked and training launches in attn_fwd_pipe16wm.hip).
// One wave per SIMD (the O accumulator alone takes DK registers per lane, and
// the compiler parks what does not fit in the accumulation registers), K/V
// tiles straight into LDS with padded rows (no swizzle above 128), 32-key
// tiles, and K columns past D zeroed through the load offsets (free: the
// offsets are fixed for the sweep).  Against the plain double-buffered kernel
// of attn_fwd_mfma16.h, same MI355X run, bit-identical outputs: bf16
// [1,16,4096,4096,256] 420 -> 333 us, causal 237 -> 184 us; fp16
// [2,16,2048,2048,160] 140 -> 103 us; bf16 [1,32/8,4096,4096,192] 553 ->
// 454 us; fp16 [1,8,1024,8192,256] (key-split) 149 -> 127 us.
#include "attn_fwd_pipe16.h"

namespace cmpext3 {

namespace {

template <typename T, int DK, bool CAUSAL, bool PRESCALE>
hipError_t launch_wide_dk(const FwdParams& p, const SplitArgs& sa, hipStream_t s) {
  return launch_pipe16_cfg<T, DK, 4, 32, 1, CAUSAL, PRESCALE, 1 | 8 | 256>(p, sa, s);
}

template <typename T, bool CAUSAL, bool PRESCALE>
hipError_t launch_wide(const FwdParams& p, const SplitArgs& sa, int dk, hipStream_t s) {
  switch (dk) {
    case 160: return launch_wide_dk<T, 160, CAUSAL, PRESCALE>(p, sa, s);
    case 192: return launch_wide_dk<T, 192, CAUSAL, PRESCALE>(p, sa, s);
    case 256: return launch_wide_dk<T, 256, CAUSAL, PRESCALE>(p, sa, s);
  }
  return hipErrorNotSupported;
}

}  // namespace

hipError_t launch_pipe16_wide_mt(const FwdParams& p, const SplitArgs& sa, int dk, bool bf16, bool causal,
                                 hipStream_t s);

hipError_t launch_pipe16_wide(const FwdParams& p, const SplitArgs& sa, int dk, bool bf16, bool causal,
                              bool prescale, hipStream_t s) {
  // masked and training launches: attn_fwd_pipe16wm.hip (never pre-scaled)
  if (p.lse || p.mask_kind != MASK_NONE) return launch_pipe16_wide_mt(p, sa, dk, bf16, causal, s);
  if (bf16) return causal ? launch_wide<__bf16, true, false>(p, sa, dk, s) : launch_wide<__bf16, false, false>(p, sa, dk, s);
  if (prescale)
    return causal ? launch_wide<_Float16, true, true>(p, sa, dk, s) : launch_wide<_Float16, false, true>(p, sa, dk, s);
  return causal ? launch_wide<_Float16, true, false>(p, sa, dk, s) : launch_wide<_Float16, false, false>(p, sa, dk, s);
}

}  // namespace cmpext3
