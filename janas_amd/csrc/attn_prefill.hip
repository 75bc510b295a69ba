/* attn_prefill.hip - placeholder until the MFMA prefill kernel lands */
#include "attn_kernels.h"
namespace janas {
int prefill_supported(int, uint32_t) { return 0; }
uint32_t prefill_block_tokens(uint32_t) { return 64; }
hipError_t launch_prefill(int, const PrefillArgs &, hipStream_t) { return hipErrorInvalidValue; }
}
