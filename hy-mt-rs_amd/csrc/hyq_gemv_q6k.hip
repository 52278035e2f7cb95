// Batch-1 int8 GEMV kernels for Q6_K (hyq_gemv_impl.hpp).
#include "hyq_gemv_impl.hpp"

namespace hyq {
template int launch_gemv_format<Q6_K>(int mode, const GemvArgs &a, void *stream);
} // namespace hyq
