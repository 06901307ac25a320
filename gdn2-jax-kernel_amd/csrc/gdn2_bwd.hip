// GDN-2 backward on gfx950 (placeholder until the B1-B5 kernels land).
#include "gdn2_common.h"
#include "gdn2_layout.h"

namespace gdn2 {

size_t bwd_ws_bytes(size_t nchunks, int BT, int D, size_t elem) { return 0; }

template <typename T, typename TG, int BT, int D>
hipError_t launch_bwd(hipStream_t, int, int, int, const void*, const void*, const void*,
                      const void*, const void*, const void*, const float*, float, const float*,
                      const float*, void*, void*, void*, void*, void*, void*, float*,
                      const char*, char*) {
  return hipErrorNotSupported;
}

#define GDN2_INST_BWD(T, TG, BT, D)                                                        \
  template hipError_t launch_bwd<T, TG, BT, D>(                                            \
      hipStream_t, int, int, int, const void*, const void*, const void*, const void*,      \
      const void*, const void*, const float*, float, const float*, const float*, void*,    \
      void*, void*, void*, void*, void*, float*, const char*, char*);
GDN2_INST_BWD(float, float, 64, 64)
GDN2_INST_BWD(float, float, 64, 128)
GDN2_INST_BWD(bf16_t, float, 64, 64)
GDN2_INST_BWD(bf16_t, float, 64, 128)
GDN2_INST_BWD(bf16_t, float, 128, 64)
GDN2_INST_BWD(bf16_t, float, 128, 128)
GDN2_INST_BWD(bf16_t, bf16_t, 64, 64)
GDN2_INST_BWD(bf16_t, bf16_t, 64, 128)
GDN2_INST_BWD(bf16_t, bf16_t, 128, 64)
GDN2_INST_BWD(bf16_t, bf16_t, 128, 128)

}  // namespace gdn2
