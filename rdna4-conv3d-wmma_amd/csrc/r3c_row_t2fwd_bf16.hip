// r3c_row_t2fwd_bf16.hip -- bf16 instantiations of the row kernel, mode MODE_T2FWD.
#include "r3c_row.h"

namespace r3c {

bool launch_row_t2fwd_bf16(int nb, int cl, int wf, const RowArgs& a, int cus, size_t lds, hipStream_t s) {
  if (wf == 1 && cl == 2 && nb == 1) {
    launch_row_inst<bf16_tag, MODE_T2FWD, 1, 2, 1>(a, cus, lds, s);
    return true;
  }
  if (wf == 1 && cl == 2 && nb == 2) {
    launch_row_inst<bf16_tag, MODE_T2FWD, 2, 2, 1>(a, cus, lds, s);
    return true;
  }
  if (wf == 1 && cl == 2 && nb == 3) {
    launch_row_inst<bf16_tag, MODE_T2FWD, 3, 2, 1>(a, cus, lds, s);
    return true;
  }
  if (wf == 0 && cl == 2 && nb == 1) {
    launch_row_inst<bf16_tag, MODE_T2FWD, 1, 2, 0>(a, cus, lds, s);
    return true;
  }
  if (wf == 0 && cl == 2 && nb == 2) {
    launch_row_inst<bf16_tag, MODE_T2FWD, 2, 2, 0>(a, cus, lds, s);
    return true;
  }
  if (wf == 0 && cl == 2 && nb == 3) {
    launch_row_inst<bf16_tag, MODE_T2FWD, 3, 2, 0>(a, cus, lds, s);
    return true;
  }
  if (wf == 1 && cl == 1 && nb == 1) {
    launch_row_inst<bf16_tag, MODE_T2FWD, 1, 1, 1>(a, cus, lds, s);
    return true;
  }
  if (wf == 1 && cl == 1 && nb == 2) {
    launch_row_inst<bf16_tag, MODE_T2FWD, 2, 1, 1>(a, cus, lds, s);
    return true;
  }
  if (wf == 1 && cl == 1 && nb == 3) {
    launch_row_inst<bf16_tag, MODE_T2FWD, 3, 1, 1>(a, cus, lds, s);
    return true;
  }
  if (wf == 1 && cl == 0 && nb == 1) {
    launch_row_inst<bf16_tag, MODE_T2FWD, 1, 0, 1>(a, cus, lds, s);
    return true;
  }
  if (wf == 1 && cl == 0 && nb == 2) {
    launch_row_inst<bf16_tag, MODE_T2FWD, 2, 0, 1>(a, cus, lds, s);
    return true;
  }
  if (wf == 1 && cl == 0 && nb == 3) {
    launch_row_inst<bf16_tag, MODE_T2FWD, 3, 0, 1>(a, cus, lds, s);
    return true;
  }
  if (wf == 0 && cl == 1 && nb == 1) {
    launch_row_inst<bf16_tag, MODE_T2FWD, 1, 1, 0>(a, cus, lds, s);
    return true;
  }
  if (wf == 0 && cl == 1 && nb == 2) {
    launch_row_inst<bf16_tag, MODE_T2FWD, 2, 1, 0>(a, cus, lds, s);
    return true;
  }
  if (wf == 0 && cl == 1 && nb == 3) {
    launch_row_inst<bf16_tag, MODE_T2FWD, 3, 1, 0>(a, cus, lds, s);
    return true;
  }
  if (wf == 0 && cl == 0 && nb == 1) {
    launch_row_inst<bf16_tag, MODE_T2FWD, 1, 0, 0>(a, cus, lds, s);
    return true;
  }
  if (wf == 0 && cl == 0 && nb == 2) {
    launch_row_inst<bf16_tag, MODE_T2FWD, 2, 0, 0>(a, cus, lds, s);
    return true;
  }
  if (wf == 0 && cl == 0 && nb == 3) {
    launch_row_inst<bf16_tag, MODE_T2FWD, 3, 0, 0>(a, cus, lds, s);
    return true;
  }
  if (wf == 1 && cl == 2 && nb == 6) {
    launch_row_inst<bf16_tag, MODE_T2FWD, 6, 2, 1>(a, cus, lds, s);
    return true;
  }
  if (wf == 1 && cl == 1 && nb == 6) {
    launch_row_inst<bf16_tag, MODE_T2FWD, 6, 1, 1>(a, cus, lds, s);
    return true;
  }
  if (wf == 1 && cl == 0 && nb == 6) {
    launch_row_inst<bf16_tag, MODE_T2FWD, 6, 0, 1>(a, cus, lds, s);
    return true;
  }
  if (wf == 0 && cl == 2 && nb == 6) {
    launch_row_inst<bf16_tag, MODE_T2FWD, 6, 2, 0>(a, cus, lds, s);
    return true;
  }
  if (wf == 0 && cl == 1 && nb == 6) {
    launch_row_inst<bf16_tag, MODE_T2FWD, 6, 1, 0>(a, cus, lds, s);
    return true;
  }
  if (wf == 0 && cl == 0 && nb == 6) {
    launch_row_inst<bf16_tag, MODE_T2FWD, 6, 0, 0>(a, cus, lds, s);
    return true;
  }
  return false;
}

}  // namespace r3c
