// r3c_t2dx.hip -- instantiations of the register-direct ConvTranspose dX
// (r3c_t2dx.h) and its A-fragment packing.  One or two row blocks of 32 input
// channels per workgroup (more spill registers), four k-steps per stage.
#include "r3c_t2dx.h"

namespace r3c {

bool launch_t2dx(int dtype, int rb, const T2dxArgs& a, size_t lds, hipStream_t s) {
  if (dtype == DT_BF16) {
    if (rb == 1) return launch_t2dx_inst<bf16_tag, 1, 4>(a, lds, s), true;
    if (rb == 2) return launch_t2dx_inst<bf16_tag, 2, 4>(a, lds, s), true;
  } else {
    if (rb == 1) return launch_t2dx_inst<f16_tag, 1, 4>(a, lds, s), true;
    if (rb == 2) return launch_t2dx_inst<f16_tag, 2, 4>(a, lds, s), true;
  }
  return false;
}

void launch_t2dx_pack(const T2dxPackArgs& a, hipStream_t s) {
  hipLaunchKernelGGL(t2dx_pack_kernel, dim3((unsigned)((a.total + 255) / 256)), dim3(256), 0, s, a);
}

}  // namespace r3c
