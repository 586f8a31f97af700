// GPT-OSS MXFP4 MoE — placeholder until the grouped-expert kernels land.
#include "nnq_device.h"
#include "nnq_internal.h"
#include <cstring>

namespace nnq {
size_t moe_scratch_bytes(int64_t, int64_t, int64_t, int64_t, int) { return 16; }
int launch_moe(const MoeDev &, const void *, int, int64_t, const float *, int, float, float *, uint32_t *, float *,
               void *, void *) { return (int)hipErrorNotSupported; }
int launch_moe_dequant(const MoeDev &, int64_t, float *, float *, void *) { return (int)hipErrorNotSupported; }
void moe_repack(const uint8_t *packed, int64_t E, int64_t K, int64_t N, uint8_t *dst) { std::memcpy(dst, packed, (size_t)E * K * N / 2); }
}  // namespace nnq
