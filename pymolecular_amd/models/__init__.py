"""Mirror of the reference's ``models`` package (only the EGNN layer family exists there)."""
