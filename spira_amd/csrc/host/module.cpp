// The `spira_amd.nn.functional._C` extension module: the same function names
// and argument order as the reference's pybind module
// (source/setup.py:129, torch/common.h:17-21).
#include "host_common.h"

PYBIND11_MODULE(_C, m) {
  m.doc() = "spira sparse-convolution extension for MI355X (gfx950)";
  spira_host::register_coords(m);
  spira_host::register_mapping(m);
  spira_host::register_conv(m);
}
