// Tensor-product kernel instantiations with in1 rank L1 = 3 (split for parallel builds).
#include "fc_tp_impl.h"
namespace fc {
int dispatch_tp_l3(int l2, int lo, bool sym, const TPArgs& g, bool conv, bool bwd, hipStream_t s) {
  return dispatch_tp_for<3>(l2, lo, sym, g, conv, bwd, s);
}
}  // namespace fc
