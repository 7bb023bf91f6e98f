// Single translation unit of the gfx950 code object embedded in libbrik.so.
#include "dequant.hip"
#include "gemv.hip"
#include "gemm.hip"
#include "topk.hip"
#include "quantize.hip"
#include "conv.hip"
#include "f16w.hip"
