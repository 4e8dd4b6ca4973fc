// Contiguous-layout decode instantiations: 64-dim f16 values, passthrough (heavy-block) values.
#include "ssq_decode_contig.h"

SSQ_CONTIG_UNIT(ssq_contig_64_f16_mixed) { return contig_mixed<4, SSQ_F16, true>(cp, pl, st); }
