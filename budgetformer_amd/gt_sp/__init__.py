"""Mirror of the reference's ``gt_sp`` call sites on the hot path."""
