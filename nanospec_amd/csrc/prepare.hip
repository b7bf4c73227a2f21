// Draft-slot preparation: labels, validity, position weights, previous ids and
// teacher indices for every (batch row, anchor block, slot) -- the objective inputs
// built by nanospec/dspark.py:116-127 and 143 (prepare), given sampled anchors.
//
// One thread per anchor block walks its K slots in order, so the prefix product of
// validity (cumprod over the slot axis) is a running flag.  Integer outputs are
// exact; weights are valid * exp(-slot / gamma) in fp32 (no decay when gamma <= 0).
#include "ns_internal.h"
#include "ns_profile.h"

namespace ns {
namespace {

__global__ __launch_bounds__(256) void prepare_kernel(const int64_t* __restrict__ ids,
                                                      const float* __restrict__ loss_mask,
                                                      const int64_t* __restrict__ anchors,
                                                      const uint8_t* __restrict__ keep, int64_t b, int64_t s,
                                                      int64_t nb, int64_t k, float gamma,
                                                      int64_t* __restrict__ target_ids,
                                                      int64_t* __restrict__ previous, float* __restrict__ weights,
                                                      uint8_t* __restrict__ valid,
                                                      int64_t* __restrict__ teacher_indices) {
  const int64_t blk = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (blk >= b * nb) return;
  const int64_t row = blk / nb;
  const int64_t j = blk % nb;
  const int64_t* ids_row = ids + row * s;
  const float* mask_row = loss_mask + row * s;
  const int64_t a = anchors[row * nb + j];
  const bool kept = keep[row * nb + j] != 0;
  bool alive = true;
  // the anchor token itself precedes slot 0 (dspark.py:127); anchors index ids directly
  const int64_t a_safe = a < 0 ? 0 : (a >= s ? s - 1 : a);
  int64_t prev = ids_row[a_safe];
  for (int64_t t = 0; t < k; ++t) {
    const int64_t label = a + t + 1;
    const int64_t safe = kept ? (label < s - 1 ? label : s - 1) : 0;
    const int64_t tgt = ids_row[safe];
    alive = alive && kept && label < s && mask_row[safe] > 0.5f;
    const int64_t o = blk * k + t;
    target_ids[o] = tgt;
    previous[o] = prev;
    valid[o] = alive ? 1 : 0;
    float w = alive ? 1.f : 0.f;
    if (gamma > 0.f) w *= expf(-(float)t / gamma);
    weights[o] = w;
    teacher_indices[o] = safe - 1 > 0 ? safe - 1 : 0;
    prev = tgt;
  }
}

}  // namespace

hipError_t prepare_slots(const int64_t* ids, const float* loss_mask, const int64_t* anchors, const uint8_t* keep,
                         int64_t b, int64_t s, int64_t nb, int64_t k, float gamma, int64_t* target_ids,
                         int64_t* previous, float* weights, uint8_t* valid, int64_t* teacher_indices,
                         hipStream_t st) {
  const int64_t blocks = b * nb;
  if (blocks == 0 || k == 0) return hipSuccess;
  NS_TIMED("prepare_slots", st);
  hipLaunchKernelGGL(prepare_kernel, dim3((unsigned)((blocks + 255) / 256)), dim3(256), 0, st, ids, loss_mask,
                     anchors, keep, b, s, nb, k, gamma, target_ids, previous, weights, valid, teacher_indices);
  return hipGetLastError();
}

}  // namespace ns
