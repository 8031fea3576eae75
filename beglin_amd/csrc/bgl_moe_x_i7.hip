// bgl_moe_x_i7.hip -- one kernel instance of the MoE gather, k_moe_x2<8, true> (device code in bgl_moe_x.h).
#include "bgl_moe_x.h"

template <int NWMAX, bool SEG1>
void moe_x2_go(dim3 g, dim3 b, size_t lds, hipStream_t st, const MoePair &P) {
    hipLaunchKernelGGL((k_moe_x2<NWMAX, SEG1>), g, b, lds, st, P);
}

template void moe_x2_go<8, true>(dim3, dim3, size_t, hipStream_t, const MoePair &);
