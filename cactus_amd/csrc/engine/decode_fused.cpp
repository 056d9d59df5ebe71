// decode_fused.cpp -- decode-step path selection of QwenModel.
#include "fused.h"

namespace cactus {

FusedDecoder::FusedDecoder(QwenModel& m) : m_(m) {}
FusedDecoder::~FusedDecoder() = default;
uint32_t FusedDecoder::step(uint32_t token) {
    (void)token;
    throw std::runtime_error("fused decode path is not built");
}

uint32_t fused_decode(QwenModel& m, FusedDecoder& f, uint32_t token) {
    (void)m;
    return f.step(token);
}

void QwenModel::set_decode_mode(int mode) {
    if (mode != 0) throw std::runtime_error("decode mode " + std::to_string(mode) + " is not built");
    decode_mode_ = mode;
}

}  // namespace cactus
