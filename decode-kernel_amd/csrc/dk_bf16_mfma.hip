// bf16 q/out over an bf16 cache, q.k on the matrix cores. Instantiation of that
// symbol table (each table is its own translation unit, compiled in parallel).
#include "dk_launch.h"

namespace dk {
template const void* pass1_symbol_16<BF16, true>(int, int, int, bool);
}  // namespace dk
