// Kernel launchers replaced by counters, for the host-only sanitizer build of
// libmxq's C ABI (tests/test_sanitize.py): every argument check in
// mxq_api.cpp runs as in the real library, and a call that passes them is
// counted instead of launched. Test infrastructure only.
#include "../../wuxianhuabu_amd/csrc/mxq_internal.hpp"

int g_launches = 0;

namespace mxq {
namespace detail {
static hipError_t count() {
  ++g_launches;
  return hipSuccess;
}
hipError_t launch_pack(const uint8_t*, int64_t, int64_t, int, uint32_t*, hipStream_t) {
  return count();
}
hipError_t launch_unpack(const uint32_t*, int64_t, int64_t, int, uint8_t*, hipStream_t) {
  return count();
}
hipError_t launch_quantize(const void*, int, int64_t, int64_t, int, int, int, uint32_t*, void*,
                           void*, int, hipStream_t) {
  return count();
}
hipError_t launch_dequantize(const uint32_t*, const void*, const void*, int, int64_t, int64_t,
                             int, int, void*, int, hipStream_t) {
  return count();
}
hipError_t launch_tile(const uint32_t*, const uint16_t*, const uint16_t*, int64_t, int64_t, int,
                       int, bool, void*, hipStream_t) {
  return count();
}
hipError_t launch_untile(const void*, int64_t, int64_t, int, int, bool, uint32_t*, uint16_t*,
                         uint16_t*, hipStream_t) {
  return count();
}
hipError_t launch_qmv(const uint16_t*, int, int, const uint32_t*, const uint16_t*,
                      const uint16_t*, int, int, int, const uint16_t*, uint16_t*, hipStream_t) {
  return count();
}
hipError_t launch_qmm(const uint16_t*, int, int, const uint32_t*, const uint16_t*,
                      const uint16_t*, int, int, int, const uint16_t*, uint16_t*, hipStream_t) {
  return count();
}
bool qmm_supports_bits(int bits) { return bits >= 2 && bits <= 8 && bits != 7; }
hipError_t launch_qmm_tiled(const uint16_t*, int, int, const void*, int, int, int,
                            const uint16_t*, int, const uint16_t*, const uint16_t*, int,
                            uint16_t*, hipStream_t) {
  return count();
}
hipError_t launch_qmv_tiled(const uint16_t*, int, int, const void*, int, int, int,
                            const uint16_t*, uint16_t*, hipStream_t) {
  return count();
}
hipError_t launch_norm_modscale(const uint16_t*, int64_t, int, const uint16_t*,
                                const uint16_t*, const uint16_t*, const uint32_t*, int64_t,
                                float, uint16_t*, hipStream_t) {
  return count();
}
hipError_t launch_mod_gate(const uint16_t*, const uint16_t*, int64_t, int, const uint16_t*,
                           const uint32_t*, int64_t, uint16_t*, hipStream_t) {
  return count();
}
hipError_t launch_rmsnorm_rope(const uint16_t*, int64_t, int, int, const uint16_t*, const void*,
                               const void*, int, int, float, uint16_t*, hipStream_t) {
  return count();
}
}  // namespace detail
}  // namespace mxq
