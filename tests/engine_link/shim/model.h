/* runtime/model.h for the engine build: the descriptor ABI and model globals. */
#include "plamo_model.h"
