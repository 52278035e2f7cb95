// Batch-1 int8 GEMV kernels for STQ1_0 (hyq_gemv_impl.hpp).
#include "hyq_gemv_impl.hpp"

namespace hyq {
template int launch_gemv_format<STQ1_0>(int mode, const GemvArgs &a, void *stream);
} // namespace hyq
