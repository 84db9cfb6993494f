// Persistent decode kernels for head_dim 64 (all batch tiles and row paddings).
#include "decode_persistent_kernel.h"

namespace fmlh {

int persist_launch_hd64(const PersistArgs& a, const PersistPlan& p, hipStream_t s) {
    return persist::launch_hd<64>(a, p, s);
}

}  // namespace fmlh
