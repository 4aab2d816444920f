// r3c_fwd_t2fwd.hip -- instantiations of the row kernel for ConvTranspose3d k2s2 forward.
#include "r3c_igemm_fwd.h"

namespace r3c {

bool launch_fwd_t2fwd(int dtype, int ck, int nb, const FwdArgs& a, size_t lds, hipStream_t s) {
#define R3C_CASE(T, CK, NB)                               \
  if (ck == CK && nb == NB) {                             \
    launch_fwd_inst<T, MODE_T2FWD, CK, NB, 4>(a, lds, s); \
    return true;                                          \
  }
#define R3C_CASES(T)                                                  \
  R3C_CASE(T, 8, 2) R3C_CASE(T, 8, 4) R3C_CASE(T, 8, 8)               \
  R3C_CASE(T, 16, 2) R3C_CASE(T, 16, 4) R3C_CASE(T, 16, 8)            \
  R3C_CASE(T, 24, 2) R3C_CASE(T, 24, 4) R3C_CASE(T, 24, 8)            \
  R3C_CASE(T, 32, 2) R3C_CASE(T, 32, 4) R3C_CASE(T, 32, 8)
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
