// fp16 q/out over an fp16 cache, q.k on the VALU; and the fp16 merge kernels. Instantiation of that
// symbol table (each table is its own translation unit, compiled in parallel).
#include "dk_launch.h"

namespace dk {
template const void* pass1_symbol_16<F16, false>(int, int, int, bool);
template const void* merge_symbol<F16>(int, bool);
}  // namespace dk
