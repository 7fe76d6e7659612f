// wh_dispatch.hip -- chooses the sampler engine for a call and sizes its workspace.
#include "wh_internal.h"

namespace wh {

size_t sample_workspace_bytes(int B, int V) {
  (void)V;
  return (size_t)(B > 0 ? B : 0) * 64 + 256;
}

int launch_sample(const SampleKArgs& k, const wh_sample_args* p, hipStream_t st) {
  (void)p;
  return launch_sample_exact(k, st);
}

}  // namespace wh
