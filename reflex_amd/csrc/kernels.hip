// The gfx950 code object of the quantized-matmul path: every kernel the host
// library (rfxq.cpp) resolves by name. Compiled with
//   hipcc --offload-arch=gfx950 --cuda-device-only --no-gpu-bundle-output -O3
// and embedded into librfxq.so (the counterpart of the reference's AOT image,
// build.rs:199-252 / src/aot.rs:113-160).
#include "common.hpp"
#include "dequant.hpp"
#include "gemv.hpp"
#include "quant.hpp"
#include "mmq.hpp"
#include "mmqh.hpp"
#include "moe.hpp"
#include "moe_decode.hpp"
