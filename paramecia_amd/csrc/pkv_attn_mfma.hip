// Specialised MFMA attention kernels for gfx950 (decode and prefill).
#include "pkv_internal.hpp"
#include "pkv_scalar.hpp"

namespace pkv {

int launch_attend_mfma(const AttnArgs &a, const float *k_new, const float *v_new, uint8_t *kc,
                       uint8_t *vc, int64_t t_new, Workspace &ws, hipStream_t s) {
  (void)a; (void)k_new; (void)v_new; (void)kc; (void)vc; (void)t_new; (void)ws; (void)s;
  return PKV_ERR_UNSUPPORTED;
}

}  // namespace pkv
