// bf16 q/out over an bf16 cache, q.k on the VALU; and the bf16 merge kernels. Instantiation of that
// symbol table (each table is its own translation unit, compiled in parallel).
#include "dk_launch.h"

namespace dk {
template const void* pass1_symbol_16<BF16, false>(int, int, int, bool);
template const void* merge_symbol<BF16>(int, bool);
}  // namespace dk
