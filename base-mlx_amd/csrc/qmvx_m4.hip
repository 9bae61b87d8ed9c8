// qmvx kernels for x-row tiles of 4 rows (see qmvx_kernel.h).
#define BMX_QMVX_KERNELS
#include "qmvx_kernel.h"

namespace bmx {
namespace qmvx {

int launch_m4(int mode, QmvEpilogue epi, const QmvParams& p, const Shape& sh, size_t lds, hipStream_t st) {
  return launch_mt<4>(mode, epi, p, sh, lds, st);
}

}  // namespace qmvx
}  // namespace bmx
