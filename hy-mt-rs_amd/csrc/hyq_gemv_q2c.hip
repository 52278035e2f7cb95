// Batch-1 int8 GEMV kernels for Q2_0C (hyq_gemv_impl.hpp).
#include "hyq_gemv_impl.hpp"

namespace hyq {
template int launch_gemv_format<Q2_0C>(int mode, const GemvArgs &a, void *stream);
} // namespace hyq
