// Split-KV decode launches for head dims that are not the power of two of
// their register layout (decode_kernels.hpp, MODE 1 and 2): any head_dim that
// fills whole 16-byte chunks of 16-byte aligned rows runs the chunk loads with
// the lanes past it idle (e.g. 80, 96, 112, 160, 192 in bf16); every other
// head_dim <= 256 (or rows that are only element-aligned) runs element loads
// with one query head per workgroup.  The reference takes any head_dim <= 256
// (src/flash_decode.py:55-61, :274-277: BLOCK_D = next power of two, every
// load masked by d < HEAD_DIM).  A translation unit of its own so that these
// instantiations compile beside the power-of-two ones.
#include "decode_kernels.hpp"

namespace mi {

hipError_t launch_split_padded(int32_t dtype, const DecodeArgs& a, const DecodePlan& p,
                               hipStream_t stream) {
  if (p.mode == 1) {
    switch (dtype) {
      case MI_DTYPE_BF16: return launch_split_mode<bf16_t, 1>(a, p, stream);
      case MI_DTYPE_F16: return launch_split_mode<f16_t, 1>(a, p, stream);
      default: return launch_split_mode<float, 1>(a, p, stream);
    }
  }
  switch (dtype) {
    case MI_DTYPE_BF16: return launch_split_mode<bf16_t, 2>(a, p, stream);
    case MI_DTYPE_F16: return launch_split_mode<f16_t, 2>(a, p, stream);
    default: return launch_split_mode<float, 2>(a, p, stream);
  }
}

}  // namespace mi
