// Batch-1 int8 GEMV dispatch: the kernels (hyq_gemv_impl.hpp) are
// instantiated one format per translation unit (hyq_gemv_<format>.hip) so
// that the five build in parallel.
#include <hip/hip_runtime.h>

#include "hyq_groups.hpp"
#include "hyq_internal.hpp"

namespace hyq {

template <int F> int launch_gemv_format(int mode, const GemvArgs &a, void *stream);

int isums_per_group(int fmt)
{
    switch (fmt) {
    case Q2_0C: return GroupQ2C::ISUMS;
    case STQ1_0: return GroupSTQ::ISUMS;
    case Q4_K: return GroupQ4K::ISUMS;
    case Q6_K: return GroupQ6K::ISUMS;
    case Q8_0: return GroupQ80::ISUMS;
    default: return -1;
    }
}

int launch_gemv(int fmt, int mode, const GemvArgs &a, void *stream)
{
    switch (fmt) {
    case Q2_0C: return launch_gemv_format<Q2_0C>(mode, a, stream);
    case STQ1_0: return launch_gemv_format<STQ1_0>(mode, a, stream);
    case Q4_K: return launch_gemv_format<Q4_K>(mode, a, stream);
    case Q6_K: return launch_gemv_format<Q6_K>(mode, a, stream);
    case Q8_0: return launch_gemv_format<Q8_0>(mode, a, stream);
    default: return (int)hipErrorInvalidValue;
    }
}

} // namespace hyq
