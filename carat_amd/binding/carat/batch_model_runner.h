// The MI355X runner under the reference's header path: with carat_amd/binding ahead of the
// reference's include/ directory, code written against include/carat/batch_model_runner.h
// (native_runtime_main.cpp's ContinuousScheduler among it) compiles against the drop-in.
#pragma once

#include "carat_hip_runner.hpp"
