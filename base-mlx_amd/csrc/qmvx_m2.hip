// qmvx kernels for x-row tiles of 2 rows (see qmvx_kernel.h).
#define BMX_QMVX_KERNELS
#include "qmvx_kernel.h"

namespace bmx {
namespace qmvx {

int launch_m2(int mode, QmvEpilogue epi, const QmvParams& p, const Shape& sh, size_t lds, hipStream_t st) {
  return launch_mt<2>(mode, epi, p, sh, lds, st);
}

}  // namespace qmvx
}  // namespace bmx
