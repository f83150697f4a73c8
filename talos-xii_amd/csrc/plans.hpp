// plans.hpp -- internal access to the model plans (plans.hip) for the other translation units.
#pragma once

#include "common.hpp"

namespace talos {

// The configuration of a PPO plan, or nullptr when plan is not one.
const talos_ppo_cfg* ppo_plan_cfg(talos_plan plan);

}  // namespace talos
