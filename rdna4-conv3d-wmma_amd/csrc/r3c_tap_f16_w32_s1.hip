// r3c_tap_f16_w32_s1.hip -- f16 instantiations of the k=3 tap kernel: lines of 32 positions,
// source staging mode 1 (channel-contiguous 16-byte slots).
#include "r3c_tap.h"

namespace r3c {

bool launch_tap_f16_w32_s1(int nb, int mb, int wf, const RowArgs& a, int cus, size_t lds, hipStream_t s) {
#define R3C_TAP(NB_, MB_, WF_)                                              \
  if (nb == NB_ && mb == MB_ && wf == WF_) {                                \
    launch_tap_inst<f16_tag, NB_, MB_, 1, WF_, 32>(a, cus, lds, s);   \
    return true;                                                            \
  }
  R3C_TAP(1, 4, 1)
  R3C_TAP(1, 4, 0)
  R3C_TAP(1, 2, 1)
  R3C_TAP(1, 2, 0)
  R3C_TAP(1, 1, 1)
  R3C_TAP(1, 1, 0)
  R3C_TAP(2, 2, 0)
  R3C_TAP(2, 1, 0)
  R3C_TAP(3, 2, 0)
  R3C_TAP(3, 1, 0)
#undef R3C_TAP
  return false;
}

}  // namespace r3c
