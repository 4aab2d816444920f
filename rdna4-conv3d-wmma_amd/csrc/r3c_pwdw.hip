// r3c_pwdw.hip -- instantiations of the register-direct single-tap weight
// gradient (r3c_pwdw.h): Conv3d k=1 with K blocks of 64 positions, and
// ConvTranspose k2s2 with K blocks of 16 or 32 positions (one w row).
#include "r3c_pwdw.h"

namespace r3c {

#define R3C_PWDW(T_, MODE_, TR_, TC_, NJ_)                  \
  if (mode == MODE_ && tr == TR_ && tc == TC_ && nj == NJ_) { \
    launch_pwdw_inst<T_, MODE_, TR_, TC_, NJ_>(a, s);        \
    return true;                                            \
  }
// Tile groups that fit the register file without spilling: at most three
// tiles with k=1's 64-position K blocks, at most four for ConvTranspose.
#define R3C_PWDW_TILES(T_, MODE_, NJ_) \
  R3C_PWDW(T_, MODE_, 1, 1, NJ_)       \
  R3C_PWDW(T_, MODE_, 1, 2, NJ_)       \
  R3C_PWDW(T_, MODE_, 1, 3, NJ_)       \
  R3C_PWDW(T_, MODE_, 2, 1, NJ_)       \
  R3C_PWDW(T_, MODE_, 3, 1, NJ_)
#define R3C_PWDW_ALL(T_)               \
  R3C_PWDW_TILES(T_, MODE_K1, 4)       \
  R3C_PWDW_TILES(T_, MODE_T2DW, 1)     \
  R3C_PWDW(T_, MODE_T2DW, 2, 2, 1)     \
  R3C_PWDW_TILES(T_, MODE_T2DW, 2)     \
  R3C_PWDW(T_, MODE_T2DW, 2, 2, 2)

bool launch_pwdw(int dtype, int mode, int tr, int tc, int nj, const PwdwArgs& a, hipStream_t s) {
  if (dtype == DT_BF16) {
    R3C_PWDW_ALL(bf16_tag)
  } else {
    R3C_PWDW_ALL(f16_tag)
  }
  return false;
}
#undef R3C_PWDW_ALL
#undef R3C_PWDW_TILES
#undef R3C_PWDW

}  // namespace r3c
