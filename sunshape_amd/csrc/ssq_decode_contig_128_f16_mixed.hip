// Contiguous-layout decode instantiations: 128-dim f16 values, passthrough (heavy-block) values.
#include "ssq_decode_contig.h"

SSQ_CONTIG_UNIT(ssq_contig_128_f16_mixed) { return contig_mixed<8, SSQ_F16, true>(cp, pl, st); }
