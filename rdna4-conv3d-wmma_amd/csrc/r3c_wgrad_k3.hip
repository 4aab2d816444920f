// r3c_wgrad_k3.hip -- instantiations of the weight-gradient kernel for 3x3x3 Conv3d.
#include "r3c_igemm_wgrad.h"

namespace r3c {

bool launch_wgrad_k3(int dtype, int fb, int cbw, const WgradArgs& a, size_t lds, hipStream_t s) {
#define R3C_CASE(T, FB, CBW)                               \
  if (fb == FB && cbw == CBW) {                            \
    launch_wgrad_inst<T, MODE_K3, FB, CBW>(a, lds, s);     \
    return true;                                           \
  }
#define R3C_CASES(T) R3C_CASE(T, 1, 7) R3C_CASE(T, 1, 14) R3C_CASE(T, 2, 7) R3C_CASE(T, 2, 14) R3C_CASE(T, 3, 7)
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
