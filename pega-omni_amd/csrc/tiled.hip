#include "common.h"
#include "kernels.h"
namespace omni {
int launch_prefill(const TiledArgs&, int, hipStream_t) { return -2; }
int launch_dit(const TiledArgs&, int, hipStream_t) { return -2; }
}
