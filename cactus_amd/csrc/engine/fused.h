// fused.h -- state of the fused decode path (one HIP graph per token).
#pragma once
#include "engine.h"

namespace cactus {

class FusedDecoder {
public:
    explicit FusedDecoder(QwenModel& m);
    ~FusedDecoder();
    uint32_t step(uint32_t token);

private:
    QwenModel& m_;
};

uint32_t fused_decode(QwenModel& m, FusedDecoder& f, uint32_t token);

}  // namespace cactus
