// bf16 q/out over an bf16 cache, q.k on the matrix cores: the pass-1 kernels of one head_dim (DK_HEAD_DIM, set by the build: 64, 128
// or 256) and their symbol table.
#include "dk_launch.h"

#ifndef DK_HEAD_DIM
#error "compile once per head_dim with -DDK_HEAD_DIM=64, 128 or 256"
#endif

namespace dk {
template const void* pass1_sym_g<BF16, DK_HEAD_DIM, true, false>(int, int, bool, int, bool);
}  // namespace dk
