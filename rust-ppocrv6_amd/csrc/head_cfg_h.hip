// MFMA kernels of the fp16 mode F16X2 (configurations H2 for an INT8 head, HF3 for an
// FP32 head).
#include "head_mfma.hpp"

namespace ppocr {
#define PPOCR_INST(C, G)                                                                        \
    template int stats_main_cfg<C, G>(const StatsLaunch&, int, bool, unsigned, hipStream_t);    \
    template int rows_cfg<C, G, false>(const RowsLaunch&, int, unsigned, hipStream_t);
PPOCR_INST(CFG_H2, 15)
PPOCR_INST(CFG_HF3, 15)
PPOCR_INST(CFG_H2, 10)
PPOCR_INST(CFG_HF3, 10)
#undef PPOCR_INST
}  // namespace ppocr
