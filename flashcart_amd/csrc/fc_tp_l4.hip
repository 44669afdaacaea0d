// Tensor-product kernel instantiations with in1 rank L1 = 4, compiled only into a library built
// for ranks <= 4 (FLASHCART_KERNEL_L_MAX=4 at build time; split for parallel builds).
#include "fc_tp_impl.h"
namespace fc {
#if FC_KERNEL_L_MAX >= 4
int dispatch_tp_l4(int l2, int lo, bool sym, const TPArgs& g, bool conv, bool bwd, hipStream_t s) {
  return dispatch_tp_for<4>(l2, lo, sym, g, conv, bwd, s);
}
#endif
}  // namespace fc
