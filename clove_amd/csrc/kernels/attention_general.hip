// attention_general.hip -- the attention prefill at every head dim the
// fixed-shape builds (64 and 128, flash_attention.hip) do not cover.
//
// Clove gives head_dim = dim / num_heads with no restriction (nn.rs:519,
// nn/attention.rs:47), and the lazy FlashAttention step takes it from the
// RoPE nodes (lazy.rs:1621-1690), so any D in [1, 256] runs here: the
// 16-query MFMA kernel of attention16.h with its tiles laid out for DP, the
// next size of kPads at or above D, and D itself read at run time (dims past
// D load as zero).  The pad set keeps the MFMA work within 16 dims of D up to
// 128 and within 32 above it.
#include <hip/hip_runtime.h>

#include "attention16.h"

namespace clove {
namespace k {

namespace {

template <int DP>
void launch(const AttnArgs &a, bool causal, unsigned grid, hipStream_t s) {
    if (a.D % 4 == 0) {
        if (causal) attention16_kernel<DP, true, true, true><<<grid, 512, 0, s>>>(a);
        else attention16_kernel<DP, false, true, true><<<grid, 512, 0, s>>>(a);
    } else {
        if (causal) attention16_kernel<DP, true, true, false><<<grid, 512, 0, s>>>(a);
        else attention16_kernel<DP, false, true, false><<<grid, 512, 0, s>>>(a);
    }
}

}  // namespace

void attention_prefill_general(const AttnArgs &a, bool causal, unsigned grid, hipStream_t s) {
    const int D = a.D;
    if (D <= 16) launch<16>(a, causal, grid, s);
    else if (D <= 32) launch<32>(a, causal, grid, s);
    else if (D <= 48) launch<48>(a, causal, grid, s);
    else if (D <= 64) launch<64>(a, causal, grid, s);
    else if (D <= 80) launch<80>(a, causal, grid, s);
    else if (D <= 96) launch<96>(a, causal, grid, s);
    else if (D <= 112) launch<112>(a, causal, grid, s);
    else if (D <= 128) launch<128>(a, causal, grid, s);
    else if (D <= 160) launch<160>(a, causal, grid, s);
    else if (D <= 192) launch<192>(a, causal, grid, s);
    else if (D <= 224) launch<224>(a, causal, grid, s);
    else launch<256>(a, causal, grid, s);
}

}  // namespace k
}  // namespace clove
