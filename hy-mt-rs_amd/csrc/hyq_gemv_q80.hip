// Batch-1 int8 GEMV kernels for Q8_0 (hyq_gemv_impl.hpp).
#include "hyq_gemv_impl.hpp"

namespace hyq {
template int launch_gemv_format<Q8_0>(int mode, const GemvArgs &a, void *stream);
} // namespace hyq
