// Instantiations of the Viterbi launcher for parity mode 3 (S = 1024, every label count).
#include "tcq_launch.h"
namespace ltq {
template int launch<10, 3, 4>(const TcqArgs&, hipStream_t);
template int launch<10, 3, 8>(const TcqArgs&, hipStream_t);
template int launch<10, 3, 16>(const TcqArgs&, hipStream_t);
template int launch<10, 3, 32>(const TcqArgs&, hipStream_t);
}  // namespace ltq
