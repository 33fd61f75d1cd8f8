/**
 * @file optimizer.hpp
 * @brief Optimizer base (ref: include/CppNet/optimizers/optimizer.hpp:20-21).
 *
 * update() keeps the reference signature.  In this backend the parameter and
 * gradient pointers are DEVICE pointers (the layers' HBM-resident state);
 * passing host memory is rejected with std::invalid_argument.
 * begin_group()/end_group() let a caller (SequentialModel::update) gather the
 * updates of many tensors into one fused launch.
 */
#ifndef CPPNET_OPTIMIZERS_OPTIMIZER_HPP
#define CPPNET_OPTIMIZERS_OPTIMIZER_HPP

#include <cstdint>
#include <vector>

namespace CppNet
{
    namespace Optimizers
    {
        class Optimizer
        {
        public:
            virtual void update(float* weights, const float* gradients, int size,
                                float learning_rate) = 0;
            virtual void update(float* weights, const float* gradients, int64_t size,
                                float learning_rate)
            {
                update(weights, gradients, static_cast<int>(size), learning_rate);
            }
            virtual void begin_group() {}
            virtual void end_group() {}
            virtual ~Optimizer() = default;

            // Undoes the host-side bookkeeping (step counts) of updates the
            // device withheld after a persistent recurrence launch gave up
            // (cnhip_recurrence_fault_check); the device left their tensors
            // unchanged.  Called by the optimizer before each launch and by
            // the training session when it reports such a fault.
            virtual void reconcile_withheld() {}

            // Checkpoint support (Utils::save_checkpoint; no counterpart in the
            // reference, whose model files hold weights only).  kind_code()
            // names the algorithm in a checkpoint (-1: none saved),
            // state_tensors() is how many n-float tensors it keeps per
            // parameter.  get_state fills host copies of the state kept for
            // the parameter at `weights` and its step count, and returns false
            // when that parameter has none yet; set_state installs such a
            // state (synchronously).
            virtual int kind_code() const { return -1; }
            virtual int state_tensors() const { return 0; }
            virtual bool get_state(const float* /*weights*/, int64_t /*n*/,
                                   std::vector<std::vector<float>>& /*tensors*/, int& /*t*/) const
            {
                return false;
            }
            virtual void set_state(const float* /*weights*/, int64_t /*n*/,
                                   const std::vector<std::vector<float>>& /*tensors*/, int /*t*/)
            {
            }
        };
    } // namespace Optimizers
} // namespace CppNet
#endif
