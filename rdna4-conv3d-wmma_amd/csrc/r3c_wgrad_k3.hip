// r3c_wgrad_k3.hip -- instantiations of the weight-gradient kernel, mode MODE_K3.
#include "r3c_wgrad.h"

namespace r3c {

// (cl, fl) pairs: G by 16-byte channel vectors or scalars (cl 1 / 0), F from a
// [position][channel] or channel-major tile (fl 0 / 1); fl 3 stages both from
// w-contiguous (NCDHW) sources and ignores cl (the host passes 0).
#define R3C_WG_K3(T_, CBW_, CL_, FL_)                          \
  if (cbw == CBW_ && cl == CL_ && fl == FL_) {                 \
    launch_wgrad_inst<T_, MODE_K3, CBW_, CL_, FL_>(a, lds, s); \
    return true;                                               \
  }
#define R3C_WG_K3_ALL(T_)   \
  R3C_WG_K3(T_, 1, 1, 0)    \
  R3C_WG_K3(T_, 2, 1, 0)    \
  R3C_WG_K3(T_, 3, 1, 0)    \
  R3C_WG_K3(T_, 4, 1, 0)    \
  R3C_WG_K3(T_, 1, 0, 0)    \
  R3C_WG_K3(T_, 2, 0, 0)    \
  R3C_WG_K3(T_, 3, 0, 0)    \
  R3C_WG_K3(T_, 4, 0, 0)    \
  R3C_WG_K3(T_, 1, 1, 1)    \
  R3C_WG_K3(T_, 2, 1, 1)    \
  R3C_WG_K3(T_, 3, 1, 1)    \
  R3C_WG_K3(T_, 4, 1, 1)    \
  R3C_WG_K3(T_, 1, 0, 1)    \
  R3C_WG_K3(T_, 2, 0, 1)    \
  R3C_WG_K3(T_, 3, 0, 1)    \
  R3C_WG_K3(T_, 4, 0, 1)    \
  R3C_WG_K3(T_, 1, 0, 3)    \
  R3C_WG_K3(T_, 2, 0, 3)    \
  R3C_WG_K3(T_, 3, 0, 3)    \
  R3C_WG_K3(T_, 4, 0, 3)

bool launch_wgrad_k3_bf16(int cbw, int cl, int fl, const WgArgs& a, size_t lds, hipStream_t s) {
  R3C_WG_K3_ALL(bf16_tag)
  return false;
}
bool launch_wgrad_k3_f16(int cbw, int cl, int fl, const WgArgs& a, size_t lds, hipStream_t s) {
  R3C_WG_K3_ALL(f16_tag)
  return false;
}
#undef R3C_WG_K3_ALL
#undef R3C_WG_K3

}  // namespace r3c
