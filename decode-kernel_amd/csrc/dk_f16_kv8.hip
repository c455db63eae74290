// fp16 q/out over an fp8 (E4M3) cache, q.k on the VALU. Instantiation of that
// symbol table (each table is its own translation unit, compiled in parallel).
#include "dk_launch.h"

namespace dk {
template const void* pass1_symbol_kv8<F16, false>(int, int, int, bool);
}  // namespace dk
