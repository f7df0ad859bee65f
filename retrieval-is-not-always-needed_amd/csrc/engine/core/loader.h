// .rinn model files (rina-engine/src/loader.cpp:14-152, written by
// tools/convert_llama_to_rinn.py:97-123).
#pragma once
#include <string>
#include "core/config.h"
#include "core/tensor.h"

// load_model of loader.cpp:149-152: path is the file or a directory holding
// weights.rinn.  Reads the 512-byte header, the JSON config and the tensor
// index, uploads every tensor to device memory the map owns, and returns
// false with *err set on a missing file, a bad magic, a truncated file or
// a quant type the reader does not take (FP32, Q4_0, Q4_0F as the
// reference's loader; nothing is left allocated then).
bool load_rinn(const std::string& path, ModelConfig& cfg, TensorMap& tensors, std::string* err);
