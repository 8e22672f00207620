/* runtime/draft.h for the engine build: the in-process proposer. */
#include "plamo_draft.h"
