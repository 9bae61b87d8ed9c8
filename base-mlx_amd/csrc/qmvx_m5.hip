// qmvx kernels for x-row tiles of 5 rows (see qmvx_kernel.h).
#define BMX_QMVX_KERNELS
#include "qmvx_kernel.h"

namespace bmx {
namespace qmvx {

int launch_m5(int mode, QmvEpilogue epi, const QmvParams& p, const Shape& sh, size_t lds, hipStream_t st) {
  return launch_mt<5>(mode, epi, p, sh, lds, st);
}

}  // namespace qmvx
}  // namespace bmx
