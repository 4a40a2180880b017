// velox_hip_runner -- the generic runner: any builtin model (--model), .vlx source (--model-file) or
// checkpoint (--weights); the argv, report and flow are velox_hip_runner_main's (vx_runner.cpp).
#include "velox_hip.h"

int main(int argc, char** argv) { return velox_hip_runner_main(argc, argv, nullptr, nullptr); }
