// r3c_wgrow.hip -- instantiations of the row-walking k=3 weight-gradient kernel.
#include "r3c_wgrow.h"

namespace r3c {

namespace {
template <int WL>
bool launch_wl(int dtype, int gcw, const WgArgs& a, hipStream_t s) {
  const bool bf = dtype == DT_BF16;
  switch (gcw) {
    case 8: bf ? launch_wgrow_inst<bf16_tag, 8, WL>(a, s) : launch_wgrow_inst<f16_tag, 8, WL>(a, s); return true;
    case 16: bf ? launch_wgrow_inst<bf16_tag, 16, WL>(a, s) : launch_wgrow_inst<f16_tag, 16, WL>(a, s); return true;
    case 24: bf ? launch_wgrow_inst<bf16_tag, 24, WL>(a, s) : launch_wgrow_inst<f16_tag, 24, WL>(a, s); return true;
    default: return false;
  }
}
}  // namespace

bool launch_wgrow(int dtype, int gcw, int w, const WgArgs& a, hipStream_t s) {
  switch (w) {
    case 32: return launch_wl<2>(dtype, gcw, a, s);
    case 64: return launch_wl<4>(dtype, gcw, a, s);
    case 128: return launch_wl<8>(dtype, gcw, a, s);
    default: return false;
  }
}

}  // namespace r3c
