// r3c_wgrad_k3.hip -- instantiations of the weight-gradient kernel, mode MODE_K3.
#include "r3c_wgrad.h"

namespace r3c {

bool launch_wgrad_k3_bf16(int cbw, const WgArgs& a, size_t lds, hipStream_t s) {
  if (cbw == 1) {
    launch_wgrad_inst<bf16_tag, MODE_K3, 1>(a, lds, s);
    return true;
  }
  if (cbw == 2) {
    launch_wgrad_inst<bf16_tag, MODE_K3, 2>(a, lds, s);
    return true;
  }
  if (cbw == 3) {
    launch_wgrad_inst<bf16_tag, MODE_K3, 3>(a, lds, s);
    return true;
  }
  if (cbw == 4) {
    launch_wgrad_inst<bf16_tag, MODE_K3, 4>(a, lds, s);
    return true;
  }
  if (cbw == 5) {
    launch_wgrad_inst<bf16_tag, MODE_K3, 5>(a, lds, s);
    return true;
  }
  if (cbw == 6) {
    launch_wgrad_inst<bf16_tag, MODE_K3, 6>(a, lds, s);
    return true;
  }
  if (cbw == 7) {
    launch_wgrad_inst<bf16_tag, MODE_K3, 7>(a, lds, s);
    return true;
  }
  return false;
}

bool launch_wgrad_k3_f16(int cbw, const WgArgs& a, size_t lds, hipStream_t s) {
  if (cbw == 1) {
    launch_wgrad_inst<f16_tag, MODE_K3, 1>(a, lds, s);
    return true;
  }
  if (cbw == 2) {
    launch_wgrad_inst<f16_tag, MODE_K3, 2>(a, lds, s);
    return true;
  }
  if (cbw == 3) {
    launch_wgrad_inst<f16_tag, MODE_K3, 3>(a, lds, s);
    return true;
  }
  if (cbw == 4) {
    launch_wgrad_inst<f16_tag, MODE_K3, 4>(a, lds, s);
    return true;
  }
  if (cbw == 5) {
    launch_wgrad_inst<f16_tag, MODE_K3, 5>(a, lds, s);
    return true;
  }
  if (cbw == 6) {
    launch_wgrad_inst<f16_tag, MODE_K3, 6>(a, lds, s);
    return true;
  }
  if (cbw == 7) {
    launch_wgrad_inst<f16_tag, MODE_K3, 7>(a, lds, s);
    return true;
  }
  return false;
}

}  // namespace r3c
