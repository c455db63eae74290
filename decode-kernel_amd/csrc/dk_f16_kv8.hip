// fp16 q/out over an fp8 (E4M3) cache: instantiation of the decode kernels' symbol table.
#include "dk_launch.h"

namespace dk {
template const void* pass1_symbol_kv8<F16>(int, int, int, bool);
}  // namespace dk
