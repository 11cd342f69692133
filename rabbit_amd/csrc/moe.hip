// moe.hip -- per-expert helpers for apply_single_expert (glm52/moe.rs:463-513).
#include "rbt_device.h"
#include "rbt_internal.h"

namespace rbt {

// rows = tokens that picked `eid`, in token order, with their weights (glm52/moe.rs:465-470: the
// first slot of each token that matches).
__global__ void k_single_rows(const int32_t *__restrict__ ids, const float *__restrict__ w, int S, int k, int eid,
                              int *__restrict__ pair_tok, float *__restrict__ pair_w, int *__restrict__ nr) {
  if (threadIdx.x != 0 || blockIdx.x != 0) return;
  int n = 0;
  for (int t = 0; t < S; t++) {
    for (int j = 0; j < k; j++) {
      if (ids[t * k + j] == eid) {
        pair_tok[n] = t;
        pair_w[n] = w[t * k + j];
        n++;
        break;
      }
    }
  }
  *nr = n;
}

// out[tok(r), d] += w_r * y[r, d] with separate roundings (glm52/moe.rs:508-512). A token
// appears at most once per expert, so rows never collide.
__global__ void k_accumulate(const float *__restrict__ y, int S, int H, const int *__restrict__ pair_tok,
                             const float *__restrict__ pair_w, const int *__restrict__ nr, float *__restrict__ out) {
  size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  int n = *nr;
  if (idx >= (size_t)n * H) return;
  int r = (int)(idx / H), d = (int)(idx % H);
  float *o = out + (size_t)pair_tok[r] * H + d;
  *o = __fadd_rn(*o, __fmul_rn(pair_w[r], y[(size_t)r * H + d]));
}

hipError_t launch_single_rows(const Ctx &c, const int32_t *ids, const float *w, int S, int k, int eid, int *pair_tok,
                              float *pair_w, int *nr) {
  launch_k(c, k_single_rows, dim3(1), dim3(64), ids, w, S, k, eid, pair_tok, pair_w, nr);
  return hipGetLastError();
}

hipError_t launch_accumulate(const Ctx &c, const float *y, int S, int H, const int *pair_tok, const float *pair_w,
                             const int *nr, float *out) {
  size_t n = (size_t)S * H;
  if (n == 0) return hipSuccess;
  launch_k(c, k_accumulate, dim3((unsigned)((n + 255) / 256)), dim3(256), y, S, H, pair_tok,
                     pair_w, nr, out);
  return hipGetLastError();
}

}  // namespace rbt
