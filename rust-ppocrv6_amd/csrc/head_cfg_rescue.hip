// MFMA kernels of the rescue passes: the rows on a precision guard's list, recomputed with
// three bf16 activation terms (exact products with int8 weights), in gather mode.
#include "head_mfma.hpp"

namespace ppocr {
template int stats_gather_cfg<CFG_Q3, 15>(const StatsLaunch&, unsigned, hipStream_t);
template int stats_gather_cfg<CFG_Q3, 10>(const StatsLaunch&, unsigned, hipStream_t);
template int rows_cfg<CFG_Q3, 15, true>(const RowsLaunch&, int, unsigned, hipStream_t);
template int rows_cfg<CFG_Q3, 10, true>(const RowsLaunch&, int, unsigned, hipStream_t);
}  // namespace ppocr
