// Instantiations of the decode kernels for one input dtype and one rot flag, chosen by the build
// (-DKUSH_INST_IN=float | _Float16 | kush::bf16_t, -DKUSH_INST_ROT=0 | 1): every (head_dim, bits, waves)
// configuration whose page ring fits in LDS, as the entry points in kush_decode.hip dispatch them.
#define KUSH_DECODE_INSTANTIATE
#include "kush_decode.h"

#if !defined(KUSH_INST_IN) || !defined(KUSH_INST_ROT)
#error "build with -DKUSH_INST_IN=<dtype> -DKUSH_INST_ROT=<0|1>"
#endif

namespace kush {
namespace {

template <int D, int BITS, int NW>
void* launcher() {
    if constexpr (decode_fits<D, BITS, NW>())
        return reinterpret_cast<void*>(&launch_decode<D, BITS, KUSH_INST_IN, NW, (KUSH_INST_ROT != 0)>);
    else
        return nullptr;
}

// taking their addresses instantiates the launchers (and their kernels) in this object
__attribute__((used)) void* const launchers[] = {
    launcher<64, 4, 2>(),  launcher<64, 4, 4>(),  launcher<64, 4, 8>(),  launcher<64, 8, 2>(),  launcher<64, 8, 4>(),
    launcher<64, 8, 8>(),  launcher<128, 4, 2>(), launcher<128, 4, 4>(), launcher<128, 4, 8>(), launcher<128, 8, 2>(),
    launcher<128, 8, 4>(), launcher<128, 8, 8>(), launcher<256, 4, 2>(), launcher<256, 4, 4>(), launcher<256, 4, 8>(),
    launcher<256, 8, 2>(), launcher<256, 8, 4>(), launcher<256, 8, 8>()};

}  // namespace
}  // namespace kush

#ifdef KUSH_TIMELINE
// Timeline build only: copies the first `rows` rows (TIMELINE_COLS int64 each) of this unit's
// timeline records to host memory `dst` (kush_decode.h, KUSH_TIMELINE). 0 on success, else the HIP error code.
extern "C" int kush_timeline_read(void* dst, int64_t rows) {
    if (rows < 0 || rows > kush::TIMELINE_ROWS) return (int)hipErrorInvalidValue;
    const size_t bytes = (size_t)rows * kush::TIMELINE_COLS * sizeof(long long);
    return (int)hipMemcpyFromSymbol(dst, HIP_SYMBOL(kush::g_timeline), bytes, 0, hipMemcpyDeviceToHost);
}
#endif
