// dg_count.hip -- the count kernel (search_kernel<0>) in a translation unit of its own,
// so that it can be compiled under its own instruction-scheduling strategy (build.py):
// the kernel's sweep loop is bound by VALU issue, and the ILP-oriented scheduler orders
// it better than the default, while the default suits the store-bound write kernels.
#define DG_COUNT_TU 1
#include "dg_graph.hip"
