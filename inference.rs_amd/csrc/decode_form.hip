// qmm_decode_form: the decode kernel form the plain matvec's persistent route takes for one weight type, row length
// and column count, from the same decode_form() the launchers call (no counterpart in the reference; nothing is
// launched).  For tests of the guard choice on the CPU.
#include "mmvq.h"

namespace {

template <class U>
int form_of(int ncols_x, int nc, int *out) {
  const int units = U::units(ncols_x);
  const DecodeForm f = decode_form<U>(units, nc);
  out[0] = f.kernel;
  out[1] = f.s;
  out[2] = f.full ? 1 : 0;
  out[3] = units;
  return 0;
}

template <int T, int F>
int form_t(int ncols_x, int nc, int *out) {
  return form_of<typename decode_units<T, F>::pairs>(ncols_x, nc, out);
}

}  // namespace

// out[0] kernel (0 k_mmvq_p, 1 k_mmvq_p2, 2 k_mmvq in passes), out[1] units per lane it holds, out[2] 1 if it reads
// every unit unguarded, out[3] the row's units.  act_q8_0 selects the 32-value types' _q8_0 entries.  Returns 0, or
// -1 with the error recorded for arguments the launchers would refuse.
extern "C" int qmm_decode_form(int type, int ncols_x, int nc, int act_q8_0, int *out) {
  const int64_t bs = qmm_block_size(type);
  if (!out || bs == 0 || ncols_x <= 0 || ncols_x % bs != 0 || nc < 1 || nc > 8) {
    qmm_set_error("decode_form: type=%d ncols_x=%d nc=%d", type, ncols_x, nc);
    return -1;
  }
  if (act_q8_0) {
    switch (type) {
      case QMM_TYPE_Q8_0: return form_t<QMM_TYPE_Q8_0, kActQ8_0>(ncols_x, nc, out);
      case QMM_TYPE_Q4_0: return form_t<QMM_TYPE_Q4_0, kActQ8_0>(ncols_x, nc, out);
      case QMM_TYPE_Q5_0: return form_t<QMM_TYPE_Q5_0, kActQ8_0>(ncols_x, nc, out);
      default: break;
    }
  } else {
    switch (type) {
      case QMM_TYPE_Q8_0: return form_t<QMM_TYPE_Q8_0, kActSlots>(ncols_x, nc, out);
      case QMM_TYPE_Q4_0: return form_t<QMM_TYPE_Q4_0, kActSlots>(ncols_x, nc, out);
      case QMM_TYPE_Q5_0: return form_t<QMM_TYPE_Q5_0, kActSlots>(ncols_x, nc, out);
      case QMM_TYPE_Q4K: return form_t<QMM_TYPE_Q4K, kActSlots>(ncols_x, nc, out);
      case QMM_TYPE_Q5K: return form_t<QMM_TYPE_Q5K, kActSlots>(ncols_x, nc, out);
      case QMM_TYPE_Q6K: return form_t<QMM_TYPE_Q6K, kActSlots>(ncols_x, nc, out);
      case QMM_TYPE_IQ4_XS: return form_t<QMM_TYPE_IQ4_XS, kActSlots>(ncols_x, nc, out);
      default: break;
    }
  }
  qmm_set_error("decode_form: no decode matvec for type %d (act_q8_0=%d)", type, act_q8_0);
  return -1;
}
