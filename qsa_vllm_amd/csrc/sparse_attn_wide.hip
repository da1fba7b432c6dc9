// The combined decode selection + attention kernel for logits buffers wider
// than 2048 columns (select_attend_kernel<..., WIDE>), in a code object of its
// own: sparse_attn.hip compiled with QSA_ATTN_WIDE_UNIT keeps only the device
// code and qsa_attn_launch_fused_wide, which the library's
// qsa_decode_select_attention calls for such buffers.
#define QSA_ATTN_WIDE_UNIT 1
#include "sparse_attn.hip"
