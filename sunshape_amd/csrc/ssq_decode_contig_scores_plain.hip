// Contiguous-layout decode instantiations: scores only (no values), byte codes with or without a mask, 4- and 6-bit packed codes.
#include "ssq_decode_contig.h"

SSQ_CONTIG_UNIT(ssq_contig_scores_plain) { return contig_plain<4, SSQ_BF16, false>(cp, pl, st); }
