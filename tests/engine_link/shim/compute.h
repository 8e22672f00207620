/* runtime/compute.h for the engine build: the hook storage. */
#include "plamo_compute.h"
