// P == 8 kernel (n = 5..8).
#include "fh_kernels.h"

namespace fh {

hipError_t launch_oct(const ExpmArgs& args, int dtype, bool pair, hipStream_t stream) {
  return launch_generic(args, dtype, 8, pair, stream);
}

}  // namespace fh
