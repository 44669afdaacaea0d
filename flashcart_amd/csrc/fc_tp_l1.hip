// Tensor-product kernel instantiations with in1 rank L1 = 1 (split for parallel builds).
#include "fc_tp_impl.h"
namespace fc {
int dispatch_tp_l1(int l2, int lo, bool sym, const TPArgs& g, bool conv, bool bwd, hipStream_t s) {
  return dispatch_tp_for<1>(l2, lo, sym, g, conv, bwd, s);
}
}  // namespace fc
