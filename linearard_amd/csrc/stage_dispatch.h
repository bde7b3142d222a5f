// Switch helpers mapping runtime padded head dims to template instances.
#pragma once

#define LARD_DP_CASES(X, ...) \
  X(16, __VA_ARGS__)          \
  X(32, __VA_ARGS__)          \
  X(64, __VA_ARGS__)          \
  X(128, __VA_ARGS__)         \
  X(256, __VA_ARGS__)
