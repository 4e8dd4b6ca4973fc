// Contiguous-layout decode instantiations: scores only (no values), passthrough (heavy-block) values.
#include "ssq_decode_contig.h"

SSQ_CONTIG_UNIT(ssq_contig_scores_mixed) { return contig_mixed<4, SSQ_BF16, false>(cp, pl, st); }
