// r3c_wgrad_k1t2.hip -- instantiations of the weight-gradient kernel for 1x1x1
// Conv3d and ConvTranspose3d k2s2.
#include "r3c_igemm_wgrad.h"

namespace r3c {

bool launch_wgrad_k1(int dtype, int fb, int cbw, const WgradArgs& a, size_t lds, hipStream_t s) {
#define R3C_CASE(T, FB, CBW)                               \
  if (fb == FB && cbw == CBW) {                            \
    launch_wgrad_inst<T, MODE_K1, FB, CBW>(a, lds, s);     \
    return true;                                           \
  }
#define R3C_CASES(T) R3C_CASE(T, 1, 1) R3C_CASE(T, 2, 1) R3C_CASE(T, 3, 1)
  if (dtype == DT_BF16) {
    R3C_CASES(bf16_tag)
  } else {
    R3C_CASES(f16_tag)
  }
#undef R3C_CASES
#undef R3C_CASE
  return false;
}

bool launch_wgrad_t2(int dtype, int fb, int cbw, const WgradArgs& a, size_t lds, hipStream_t s) {
#define R3C_CASE(T, FB, CBW)                               \
  if (fb == FB && cbw == CBW) {                            \
    launch_wgrad_inst<T, MODE_T2DW, FB, CBW>(a, lds, s);   \
    return true;                                           \
  }
#define R3C_CASES(T)                                                         \
  R3C_CASE(T, 1, 2) R3C_CASE(T, 1, 4) R3C_CASE(T, 1, 7)                      \
  R3C_CASE(T, 2, 2) R3C_CASE(T, 2, 4) R3C_CASE(T, 2, 7)                      \
  R3C_CASE(T, 3, 2) R3C_CASE(T, 3, 4) R3C_CASE(T, 3, 7)
  if (dtype == DT_BF16) {
    R3C_CASES(bf16_tag)
  } else {
    R3C_CASES(f16_tag)
  }
#undef R3C_CASES
#undef R3C_CASE
  return false;
}

}  // namespace r3c
