// bgl_moe_x_i2.hip -- one kernel instance of the MoE gather, k_moe_x<false, 16, 64> (device code in bgl_moe_x.h).
#include "bgl_moe_x.h"

template <bool SEG, int NWMAX, int TR>
void moe_x_go(dim3 g, dim3 b, size_t lds, hipStream_t st, const MoeTask &Mt) {
    hipLaunchKernelGGL((k_moe_x<SEG, NWMAX, TR>), g, b, lds, st, Mt);
}

template void moe_x_go<false, 16, 64>(dim3, dim3, size_t, hipStream_t, const MoeTask &);
