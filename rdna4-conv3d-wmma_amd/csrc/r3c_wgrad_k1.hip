// r3c_wgrad_k1.hip -- instantiations of the weight-gradient kernel, mode MODE_K1.
#include "r3c_wgrad.h"

namespace r3c {

bool launch_wgrad_k1_bf16(int cbw, int cl, int fl, const WgArgs& a, size_t lds, hipStream_t s) {
  if (cbw == 1 && cl == 1 && fl == 0) {
    launch_wgrad_inst<bf16_tag, MODE_K1, 1, 1, 0>(a, lds, s);
    return true;
  }
  if (cbw == 1 && cl == 0 && fl == 0) {
    launch_wgrad_inst<bf16_tag, MODE_K1, 1, 0, 0>(a, lds, s);
    return true;
  }
  if (cbw == 1 && cl == 1 && fl == 1) {
    launch_wgrad_inst<bf16_tag, MODE_K1, 1, 1, 1>(a, lds, s);
    return true;
  }
  if (cbw == 1 && cl == 0 && fl == 1) {
    launch_wgrad_inst<bf16_tag, MODE_K1, 1, 0, 1>(a, lds, s);
    return true;
  }
  if (cbw == 1 && cl == 1 && fl == 2) {
    launch_wgrad_inst<bf16_tag, MODE_K1, 1, 1, 2>(a, lds, s);
    return true;
  }
  return false;
}
bool launch_wgrad_k1_f16(int cbw, int cl, int fl, const WgArgs& a, size_t lds, hipStream_t s) {
  if (cbw == 1 && cl == 1 && fl == 0) {
    launch_wgrad_inst<f16_tag, MODE_K1, 1, 1, 0>(a, lds, s);
    return true;
  }
  if (cbw == 1 && cl == 0 && fl == 0) {
    launch_wgrad_inst<f16_tag, MODE_K1, 1, 0, 0>(a, lds, s);
    return true;
  }
  if (cbw == 1 && cl == 1 && fl == 1) {
    launch_wgrad_inst<f16_tag, MODE_K1, 1, 1, 1>(a, lds, s);
    return true;
  }
  if (cbw == 1 && cl == 0 && fl == 1) {
    launch_wgrad_inst<f16_tag, MODE_K1, 1, 0, 1>(a, lds, s);
    return true;
  }
  if (cbw == 1 && cl == 1 && fl == 2) {
    launch_wgrad_inst<f16_tag, MODE_K1, 1, 1, 2>(a, lds, s);
    return true;
  }
  return false;
}

}  // namespace r3c
