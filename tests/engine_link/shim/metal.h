/* runtime/metal.h for the engine build: the GPU backend (runtime/metal.h:3-4
 * includes the engine's parallel.h and weight_cache.h first, as here). */
#include "parallel.h"
#include "weight_cache.h"
#include "plamo_backend.h"
