// Executed-tile counters of the counter-enabled build (compiled with -DTHERIA_TILE_COUNT into
// libtheria_sdpa_tiles.so, used only to measure causal tile skipping; the production library compiles these
// macros to nothing). A wave adds the 32 x 32 (query, key) units whose products it runs as it runs them, and
// adds its total to its kernel's device counter once, at the end (one lane, a vector atomic).
#pragma once

#ifdef THERIA_TILE_COUNT
#define THERIA_TILES_DECL unsigned theria_tile_units = 0
#define THERIA_TILES_ADD(n) (theria_tile_units += (unsigned)(n))
#define THERIA_TILES_FLUSH(counter)                                                          \
  do {                                                                                        \
    if ((threadIdx.x & 63) == 0) atomicAdd(&(counter), (unsigned long long)theria_tile_units); \
  } while (0)
#else
#define THERIA_TILES_DECL \
  do {                    \
  } while (0)
#define THERIA_TILES_ADD(n) \
  do {                      \
  } while (0)
#define THERIA_TILES_FLUSH(counter) \
  do {                              \
  } while (0)
#endif
