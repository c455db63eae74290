// fp16 instantiation of the decode kernels and their symbol tables.
#include "dk_launch.h"

namespace dk {
template const void* pass1_symbol<F16>(int, int, int, bool, bool);
template const void* merge_symbol<F16>(int, bool);
}  // namespace dk
