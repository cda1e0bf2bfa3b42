// MFMA kernels of the INT8 head's bf16 modes (BF16X1 / X2 / X3: configurations Q1, Q2, Q3).
#include "head_mfma.hpp"

namespace ppocr {
#define PPOCR_INST(C, G)                                                                        \
    template int stats_main_cfg<C, G>(const StatsLaunch&, int, bool, unsigned, hipStream_t);    \
    template int rows_cfg<C, G, false>(const RowsLaunch&, int, unsigned, hipStream_t);
PPOCR_INST(CFG_Q1, 15)
PPOCR_INST(CFG_Q2, 15)
PPOCR_INST(CFG_Q3, 15)
PPOCR_INST(CFG_Q1, 10)
PPOCR_INST(CFG_Q2, 10)
PPOCR_INST(CFG_Q3, 10)
#undef PPOCR_INST
}  // namespace ppocr
