// Instantiation of the Viterbi launcher for the 256-state trellis (integer mode, 4 labels).
#include "tcq_launch.h"
namespace ltq {
template int launch<8, 2, 0, 4>(const TcqArgs&, hipStream_t);
template int launch_tb<8, 2, 0, 4>(const TcqArgs&, const TcqArgs&, hipStream_t);
}  // namespace ltq
