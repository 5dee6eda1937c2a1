/*
 * flash-train for MI355X -- runtime environment variables.
 *
 * Same variable names and meaning as the reference
 * (include/flash_train/env.h:24-48).  Each macro expands to the variable's
 * name.  Name lists are comma separated with spaces and tabs trimmed around
 * each entry; a switch is on when its trimmed value is neither empty nor "0".
 * Every variable is read once, at its first use in the process.
 */
#ifndef FTRAIN_ENV_H_
#define FTRAIN_ENV_H_

/* Allow-list of Primitive names: when set, nothing outside it is selected. */
#define FTRAIN_ENABLED_PRIMITIVES "FTRAIN_ENABLED_PRIMITIVES"

/* Deny-list of Primitive names: a listed Primitive is never selected. */
#define FTRAIN_DISABLED_PRIMITIVES "FTRAIN_DISABLED_PRIMITIVES"

/* Deny-list of Finder names: a listed Finder contributes no candidates. */
#define FTRAIN_DISABLED_FINDERS "FTRAIN_DISABLED_FINDERS"

/* Switch: when on, every Plan creation re-runs selection (no cache). */
#define FTRAIN_DISABLE_CACHE "FTRAIN_DISABLE_CACHE"

#endif
