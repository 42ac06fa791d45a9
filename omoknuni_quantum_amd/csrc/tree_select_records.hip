// The select kernels that also form the unique leaves' keys and legal counts (the kRecords
// instantiations of select_root_kernel, used for waves of at most OMQ_SELECT_RECORDS_MAX_WAVE
// simulations): tree_select.hip compiled again, as a code object of its own, so that the
// kernels without the records keep the code they have alone.
#define OMQ_SELECT_RECORDS_TU 1
#include "tree_select.hip"
