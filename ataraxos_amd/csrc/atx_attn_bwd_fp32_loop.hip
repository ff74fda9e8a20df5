// fp32 attention backward over query heads and blocks of query rows: the
// LOOP instantiations of atx_attn_bwd_fp32.hip.
#define ATX_BWD_FP32_LOOP 1
#include "atx_attn_bwd_fp32.hip"
