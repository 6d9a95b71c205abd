// Decode GEMV, y = W x (+ bias) and the multi-matrix launch, for Q4_1 / Q5_0 / Q5_1 / Q8_K / Q2_K / Q3_K / Q5_K:
// the streaming kernel of gemv_stream.h instantiated for these block types.
// Replaces _dequantize + x.astype(f32) @ W.T (draco/format/gguf.py:318-468,
// draco/runtime/cpu/kernels/generic.py:32-33) for them.
#include "gemv_stream.h"

namespace draco {

int stream_ext_plain(int qtype, bool d_last, const StreamJob& job, bool xbf16, hipStream_t s) {
  return stream_ext_dispatch<kPlain>(qtype, d_last, job, xbf16, s);
}

}  // namespace draco
