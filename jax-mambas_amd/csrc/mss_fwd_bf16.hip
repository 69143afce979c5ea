// Forward selective scan, bf16-I/O instantiations (the kernel template is in
// mss_fwd_kernel.h). A translation unit of its own so that it can be compiled with the
// ILP-maximising machine scheduler, which speeds these instantiations up and slows the
// float32 ones (jax-mambas_amd/build.py).
#include "mss_fwd_kernel.h"

namespace mss {

hipError_t launch_fwd_bf16(const FwdParams& p, int zoh, int bc_bf16, hipStream_t stream) {
  if (zoh) return bc_bf16 ? launch_fwd_z<true, bf16_t, bf16_t>(p, stream) : launch_fwd_z<true, bf16_t, float>(p, stream);
  return bc_bf16 ? launch_fwd_z<false, bf16_t, bf16_t>(p, stream) : launch_fwd_z<false, bf16_t, float>(p, stream);
}

}  // namespace mss
