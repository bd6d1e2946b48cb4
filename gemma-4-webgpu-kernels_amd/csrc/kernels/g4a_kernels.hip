// The single gfx950 code object of libg4a.so (loaded with hipModuleLoad):
// every kernel of the attention path and the projections around it,
// compiled as one translation unit.
#include "attn_decode.hip"
#include "attn_prefill.hip"
#include "norm_rope.hip"
#include "linear_q.hip"
#include "elementwise.hip"
