// synapto.hip -- GPU bulk synaptogenesis step (filled in below).
#include "layer.hpp"

namespace sili {

void synapto_step(Layer &, float, const int32_t *, const int32_t *, const float *, const float *, int64_t, int,
                  int64_t *) {
    throw_error(3, "synapto_step: not implemented yet");
}

}  // namespace sili
