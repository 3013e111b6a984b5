#pragma once

// Everything of vkml's public C++ API this build carries, for callers that
// include it whole (the reference's include/vkml/vkml.hpp, which its apps
// include: apps/vkml_bench.cpp:34, apps/vkml_run.cpp:41 there). Its chat
// templates, tokenizer and safetensors reader are outside this build; the
// request loop its apps keep in apps/generation.hpp is vkml::Session here.
#include "vkml/context.hpp"
#include "vkml/dtype.hpp"
#include "vkml/error.hpp"
#include "vkml/generation.hpp"
#include "vkml/llama.hpp"
#include "vkml/ops.hpp"
#include "vkml/sampling.hpp"
#include "vkml/tensor.hpp"
