// fk_attend.hip — the translation unit of the prefill attention, compiled
// into fk_attend.hsaco (see fk_attend.h for why it is apart).
#include "fk_attend.h"
