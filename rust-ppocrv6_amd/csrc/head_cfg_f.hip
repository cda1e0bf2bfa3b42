// MFMA kernels of the FP32 head's bf16 modes (BF16X1 / X3: configurations F1, F3).
#include "head_mfma.hpp"

namespace ppocr {
#define PPOCR_INST(C, G)                                                                        \
    template int stats_main_cfg<C, G>(const StatsLaunch&, int, bool, unsigned, hipStream_t);    \
    template int rows_cfg<C, G, false>(const RowsLaunch&, int, unsigned, hipStream_t);
PPOCR_INST(CFG_F1, 15)
PPOCR_INST(CFG_F3, 15)
PPOCR_INST(CFG_F1, 10)
PPOCR_INST(CFG_F3, 10)
#undef PPOCR_INST
}  // namespace ppocr
