// Prefill GEMM (Q4_K) — placeholder until the MFMA GEMM lands.
#include "nnq_device.h"
#include "nnq_internal.h"

namespace nnq {
size_t gemm_scratch_bytes(int64_t m, int64_t k) { return (size_t)m * k * 2 + (size_t)m * 4 + 256 + (size_t)m * (k / 32) * 4; }
int launch_gemm_q4k(const GemmArgs &, void *) { return (int)hipErrorNotSupported; }
}  // namespace nnq
