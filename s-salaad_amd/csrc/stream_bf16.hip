// Instantiations of the streaming SLR / BSR kernel (stream_kernel.h) for
// bf16 activations: every block width P, fragment depth KE and token-tile
// height MT, in both modes. One file per dtype keeps the build parallel.
#include "stream_kernel.h"

namespace ssl {

template <>
hipError_t stream_launch<DT_BF16>(int mode, int sf, int P, int KE, int MT, const GroupArgs& a,
                               int64_t blocks, hipStream_t s) {
  return stream_dispatch<DT_BF16>(mode, sf, P, KE, MT, a, blocks, s);
}

template <>
hipError_t chain_launch<DT_BF16>(int sf, int P, int MT, bool fr, const ChainArgs* a,
                             const ChainTab* tab, int64_t blocks, hipStream_t s) {
  return chain_dispatch<DT_BF16>(sf, P, MT, fr, a, tab, blocks, s);
}

}  // namespace ssl
