"""Mirror of the reference's ``utils`` call sites on the hot path."""
